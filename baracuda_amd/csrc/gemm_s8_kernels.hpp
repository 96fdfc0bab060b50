// gemm_s8_kernels.hpp -- the int8 GEMM kernels and launchers shared by the
// int8 SKU translation units (gemm_s8.hip, gemm_s8_bias.hip, gemm_s8_rrr.hip).
// Epilogues:
//   EPI_I32        D = acc (int32)
//   EPI_S8         D = sat_s8(rne(act(alpha*acc + beta*C [+ bias[n]])))
//   EPI_W8A8_BF16  D = bf16_rne((sa[m]*sw[n]) * (float)acc)
//   EPI_W8A8_F32   D = (sa[m]*sw[n]) * (float)acc
//   EPI_W8A8_F64   D = (double)(((float)sa[m]*(float)sw[n]) * (float)acc), sa / sw f64
//                  (quantized_linear_w8a8_f64: the reference narrows the f64
//                  scales to f32, computes in f32 and widens the result)
// The accumulator wraps modulo 2^32 where the reference's mma.sync
// saturates; the two agree whenever |acc| < 2^31, which holds for int8
// operands in [-127,127] whenever K < 133143.
#pragma once

#include <algorithm>
#include <type_traits>

#include "gemm_mfma.hpp"
#include "gemm_mfma2.hpp"
#include "act.hpp"

namespace bk {
namespace {

using namespace mfma;

enum Epi : int { EPI_I32 = 0, EPI_S8 = 1, EPI_W8A8_BF16 = 2, EPI_W8A8_F32 = 3, EPI_W8A8_F64 = 4 };

struct S8Args {
    int M, N, K;
    const int8_t *a; int64_t lda;
    const int8_t *b; int64_t ldb;
    const int8_t *c; int64_t ldc;
    void *d; int64_t ldd;
    float alpha, beta;
    const float *sa; const float *sw;
    const void *bias;   // [N] f32 or i32, for ACT != ACT_NONE
};

// The RCR SKUs take the CUTLASS contract for a null C: the source operand is
// D itself with D's pitch, so beta != 0 accumulates into D in place
// (gemm_s8_rcr_sm80.cu:87-89, gemm_u8_rcr_sm80.cu:77-79,
// gemm_s8_rcr_sm80_bias.cu:110-111).  Every output element's C read is made
// by the thread that stores it and feeds that store, so in place is safe.
// The RRR SKUs keep their own contract (null C: no beta term).
inline void rcr_c_defaults_to_d(S8Args &p) {
    if (p.c == nullptr) {
        p.c = static_cast<const int8_t *>(p.d);
        p.ldc = p.ldd;
    }
}

// Epilogue on one group of 4 consecutive output columns of row m.
template <int EPI, bool VecOut, int ACT = ACT_NONE, typename BiasT = float>
struct S8Epilogue {
    const S8Args &p;
    // EPI_S8, whole group of 4 columns (N % 4 == 0): the 4 result bytes.
    // HasC: beta != 0 and C given (decided once per tile by the caller).
    template <bool HasC>
    __device__ __forceinline__ uint32_t pack_s8(int m, int n0, const v4i &v) const {
        int8_t o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float z = p.alpha * (float)v[r];
            if constexpr (HasC) z += p.beta * (float)p.c[(int64_t)m * p.ldc + n0 + r];
            if constexpr (ACT != ACT_NONE) {
                z += (float)static_cast<const BiasT *>(p.bias)[n0 + r];
                z = activation<ACT>(z);
            }
            o[r] = sat_cast_s8(z);
        }
        return (uint32_t)(uint8_t)o[0] | ((uint32_t)(uint8_t)o[1] << 8) | ((uint32_t)(uint8_t)o[2] << 16) |
               ((uint32_t)(uint8_t)o[3] << 24);
    }
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
            // gemm_s8_{rcr,rrr}_sm80 epilogue: z = alpha*acc + beta*C [+ bias[n]],
            // [activation], RNE, clamp (baracuda_int8_rrr_sm80.cuh:255-305).
            int8_t *d = static_cast<int8_t *>(p.d) + (int64_t)m * p.ldd + n0;
            int8_t o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float z = p.alpha * (float)v[r];
                if (p.beta != 0.0f && p.c != nullptr && r < count)
                    z += p.beta * (float)p.c[(int64_t)m * p.ldc + n0 + r];
                if constexpr (ACT != ACT_NONE) {
                    if (r < count) z += (float)static_cast<const BiasT *>(p.bias)[n0 + r];
                    z = activation<ACT>(z);
                }
                o[r] = sat_cast_s8(z);
            }
            if (vec) {
                uint32_t w = (uint32_t)(uint8_t)o[0] | ((uint32_t)(uint8_t)o[1] << 8) |
                             ((uint32_t)(uint8_t)o[2] << 16) | ((uint32_t)(uint8_t)o[3] << 24);
                *reinterpret_cast<uint32_t *>(d) = w;
            } else {
                for (int r = 0; r < count; ++r) d[r] = o[r];
            }
        } else if constexpr (EPI == EPI_W8A8_F64) {
            const double *sa64 = reinterpret_cast<const double *>(p.sa);
            const double *sw64 = reinterpret_cast<const double *>(p.sw);
            const float sam = (float)sa64[m];
            double *d = static_cast<double *>(p.d) + (int64_t)m * p.ldd + n0;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (r < count) d[r] = (double)((sam * (float)sw64[n0 + r]) * (float)v[r]);
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
template <int EPI, bool VecOut, int ACT = ACT_NONE, typename BiasT = float>
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
    const S8Epilogue<EPI, VecOut, ACT, BiasT> epi{p};
    for_each_fragment(acc, [&](int ml, int nl, const v4i &v) { epi(m_base + ml, n_base + nl, v); });
}

// RRR (B row-major [K, N]): register-staged mainloop with B transposed into
// the shared [n][k] LDS layout.  Aligned: K % 128 == 0, N % 256 == 0,
// 16-byte A rows, 4-byte B rows.
template <bool Aligned, int ACT, typename BiasT>
__global__ __launch_bounds__(NT, 1) void gemm_s8_rrr_kernel(S8Args p) {
    __shared__ __attribute__((aligned(16))) int8_t lds[4 * LDS_TILE];
    const int tiles_m = (p.M + BM - 1) / BM;
    const int tiles_n = (p.N + BN - 1) / BN;
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m_base = tm * BM, n_base = tn * BN;
    const int tid = threadIdx.x;
    RowSet as;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int r = i * LOAD_ROWS + (tid >> 3);
        as.ptr[i] = p.a + (int64_t)min(m_base + r, p.M - 1) * p.lda;
    }
    v4i acc[TM][TN];
    mainloop_rrr<Elem::S8, !Aligned, !Aligned>(lds, as, p.b, p.ldb, p.N, n_base, p.K, acc);
    const S8Epilogue<EPI_S8, false, ACT, BiasT> epi{p};
    for_each_fragment(acc, [&](int ml, int nl, const v4i &v) { epi(m_base + ml, n_base + nl, v); });
}

template <int ACT, typename BiasT>
int32_t launch_rrr_dma(const S8Args &p, hipStream_t stream);

template <int ACT, typename BiasT>
bool launch_rrr_rows(const S8Args &p, hipStream_t stream);

template <int ACT, typename BiasT>
int32_t launch_rrr(const S8Args &p, hipStream_t stream) {
    if (launch_rrr_rows<ACT, BiasT>(p, stream)) return launch_status();
    if (launch_rrr_dma<ACT, BiasT>(p, stream) == kOk) return launch_status();
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    const bool aligned = p.K % BK == 0 && p.N % BN == 0 && p.lda % 16 == 0 && p.ldb % 4 == 0 &&
                         aligned16(p.a) && (reinterpret_cast<uintptr_t>(p.b) & 3u) == 0;
    if (aligned)
        hipLaunchKernelGGL((gemm_s8_rrr_kernel<true, ACT, BiasT>), dim3(tiles), dim3(NT), 0, stream, p);
    else
        hipLaunchKernelGGL((gemm_s8_rrr_kernel<false, ACT, BiasT>), dim3(tiles), dim3(NT), 0, stream, p);
    return launch_status();
}

// ---- split-K of a partial last round of tiles (optional workspace) ----------
// T tiles on 256 CUs leave a last round of T % 256 tiles.  When that round is
// at most half full and consists of whole tile rows, its tiles are split
// along K into `split` chunks (>= 2 stages each) run in the same launch as
// the full rounds; each chunk stores its int32 accumulators in its own
// workspace slot, and a second kernel adds a tile's slots in chunk order and
// applies the epilogue.  Integer sums are exact in any order, so the output
// is bit-identical to the unsplit kernel's.
struct TailSplit {
    int full_tiles;   // tiles of the full rounds (whole tile rows), plain path
    int tail_tiles;   // tiles of the last round, split
    int split;        // K chunks per tail tile (1: no split)
};

// Last rows of M run by gemm_s8_rcr_rows_kernel instead of a row of
// 256-row tiles (N % 16 == 0): M % 256 in [1, kRowsPathMax] (all of M when
// M <= kRowsPathMax: no tiles at all), when that row of tiles would start
// another round of tiles on the 256 CUs (it costs nothing extra when it
// fits the idle CUs of the last round).  Up to kRowsPathAlways rows always;
// up to kRowsPathMax when K % kRowsStagedSB == 0 (the staged last-rows
// kernel), otherwise only when no tail-split workspace is given.  At
// N = K = 4096 the staged pass beats the split tail round and its reduction:
// M = 100 / 128 / 4196 in 11.9 / 12.8 / 66.1 us against 22.3 / 23.0 / 71.0.
constexpr int kRowsPathMax = 128;
constexpr int kRowsPathAlways = 64;
constexpr int kRowsStagedSB = 512, kRowsStagedDepth = 2;
inline int rows_path_rows(int M, int N, int limit = kRowsPathMax) { return mfma2::last_rows_pass(M, N, limit); }

// Grids of at most kSmallTilesMax 256 x 256 tiles (under half a round on
// the 256 CUs) run 128 x 128 tiles instead (Cfg<2, 2, 128>: 4 waves of
// 64 x 64, two workgroups per CU), except that with a tail-split workspace
// a deep K (>= 4096) on fewer than 64 small tiles splits K.  W8A8, N = K =
// 4096, 8 rotated weight sets, no workspace: M = 256 / 512 / 1024 / 2048
// 56 / 56 / 56 / 55 -> 24.2 / 24.9 / 26.7 / 36.0 us (the split workspace:
// 29.9 / 32.2 / 38.2 / 52.0); 129-255 tiles stay on 256 x 256 (M = 2560 /
// 3072: 46.5 / 49.6 us against 55.1 / 59.2 with small tiles).  512 x 512 x
// 8192: small tiles 43.6 us, split 30.5.
constexpr int kSmallTilesMax = 128;
inline bool small_tiles_preferred(int M, int N, int K) {
    const int64_t t256 = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    if (t256 > kSmallTilesMax) return false;
    const int64_t t128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
    return !(t128 < 64 && K >= 4096);
}

inline TailSplit tail_split_plan(int M, int N, int K) {
    TailSplit t{0, 0, 1};
    if (M <= 0 || N <= 0 || K <= 0 || K % 128 != 0) return t;
    if (small_tiles_preferred(M, N, K)) return t;
    // the rows path takes those shapes
    if (rows_path_rows(M, N, K % kRowsStagedSB == 0 ? kRowsPathMax : kRowsPathAlways) != 0) return t;
    const int tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
    const int64_t T = (int64_t)tiles_m * tiles_n;
    const int64_t full = T / 256 * 256;
    const int64_t tail = T - full;
    if (tail == 0 || tail > 128 || full % tiles_n != 0) return t;
    const int split = std::min((int)(256 / tail), K / 128 / 2);
    if (split < 2) return t;
    return TailSplit{(int)full, (int)tail, split};
}

// int32 slot of every (tail tile, chunk): 256 x 256 accumulators.
inline size_t tail_split_workspace(int M, int N, int K) {
    const TailSplit t = tail_split_plan(M, N, K);
    return t.split > 1 ? (size_t)t.tail_tiles * t.split * 65536u * sizeof(int32_t) : 0;
}

// Rows of an operand padded to whole 256-row tiles, times its row pitch,
// fit the 32-bit buffer offsets of the LDS-DMA path.
inline bool dma_extent_ok(int rows, int64_t ld) {
    return ((int64_t)(rows + 255) / 256) * 256 * ld < (1ll << 31);
}

// Fast path: 256x256 tiles (edge tiles read zeros past M / N), K % 128 == 0,
// 16-byte aligned rows ->
// LDS-DMA mainloop, 8 waves (2 x 4) of 128 x 64, v_mfma_i32_16x16x64_i8.
typedef mfma2::Cfg<2, 4> DmaCfg;

// int8 outputs of a whole tile through LDS: each wave's 128 x 64 bytes are
// staged (8 KiB per wave; LDS is free after the mainloop's last barrier) and
// written as 16-byte row segments instead of 4-byte stores.
// Partial tiles (the M / N edge, N % 16 == 0): rows past M and 16-byte
// units past N are neither computed nor stored.
template <class P, bool HasC, bool Full, class Epi>
__device__ __forceinline__ void store_s8_tile_staged_as(const mfma2::AccTile<P> &acc, int8_t *stage0, int8_t *stage1,
                                                        const S8Args &p, int m_base, int n_base, const Epi &epi) {
    typedef typename P::Cfg C;
    const int wave = threadIdx.x >> 6;
    const int wrow = (wave / C::WAVES_N) * C::WM;
    const int wcol = (wave % C::WAVES_N) * C::WN;
    int8_t *scratch = (wave < C::WAVES / 2 ? stage0 : stage1) + (wave % (C::WAVES / 2)) * (C::WM * C::WN);
    const int ncols = min(C::WN, p.N - (n_base + wcol));
    mfma2::store_u8x4_staged<P>(
        acc, scratch,
        [&](int r, int c, const v4i &v) {
            const int m = m_base + wrow + r, n = n_base + wcol + c;
            if constexpr (Full) return epi.template pack_s8<HasC>(m, n, v);
            else return (m < p.M && n < p.N) ? epi.template pack_s8<HasC>(m, n, v) : 0u;
        },
        [&](int r) {
            return m_base + wrow + r < p.M
                       ? static_cast<int8_t *>(p.d) + (int64_t)(m_base + wrow + r) * p.ldd + n_base + wcol
                       : nullptr;
        },
        ncols);
}

// The C term and the M / N bounds decided once per tile (full: whole tile
// in range), not per element.
template <class P, class Epi>
__device__ __forceinline__ void store_s8_tile_staged(const mfma2::AccTile<P> &acc, int8_t *stage0, int8_t *stage1,
                                                     const S8Args &p, int m_base, int n_base, const Epi &epi) {
    const bool has_c = p.beta != 0.0f && p.c != nullptr;
    const bool full = m_base + P::Cfg::TB <= p.M && n_base + P::Cfg::TB <= p.N;
    if (has_c) {
        if (full) store_s8_tile_staged_as<P, true, true>(acc, stage0, stage1, p, m_base, n_base, epi);
        else store_s8_tile_staged_as<P, true, false>(acc, stage0, stage1, p, m_base, n_base, epi);
    } else {
        if (full) store_s8_tile_staged_as<P, false, true>(acc, stage0, stage1, p, m_base, n_base, epi);
        else store_s8_tile_staged_as<P, false, false>(acc, stage0, stage1, p, m_base, n_base, epi);
    }
}

// `ts`: workgroups below ts.full_tiles (all of them when ts.split == 1) run
// whole tiles; the rest run K chunks of the tail tiles (tail_split_plan) and
// store their accumulators in `slots`.
template <int EPI, bool VecOut, int ACT = ACT_NONE, typename BiasT = float, class C = DmaCfg>
__global__ __launch_bounds__(C::NT, C::NT == 256 ? 2 : 1) void gemm_s8_rcr_dma_kernel(S8Args p, TailSplit ts,
                                                                         int32_t *__restrict__ slots) {
    namespace M2 = mfma2;
    typedef M2::PolicyI8<C> P;
    __shared__ __attribute__((aligned(1024))) int8_t stage0[2 * C::OPER];
    __shared__ __attribute__((aligned(1024))) int8_t stage1[2 * C::OPER];
    // Edge tiles (M or N not a multiple of 256): operand rows past M / N
    // lie past the buffer resources' byte counts and load as zeros.
    const int tiles_n = (p.N + C::TB - 1) / C::TB;
    int tm, tn, k0 = 0, klen = p.K, chunk = -1;
    if (ts.split > 1 && (int)blockIdx.x >= ts.full_tiles) {
        const int u = blockIdx.x - ts.full_tiles, ti = u / ts.split;
        chunk = u % ts.split;
        tm = ts.full_tiles / tiles_n + ti / tiles_n;
        tn = ti % tiles_n;
        const int kt = p.K / M2::BK;
        k0 = chunk * kt / ts.split * M2::BK;
        klen = (chunk + 1) * kt / ts.split * M2::BK - k0;
    } else {
        const int tiles_m = ts.split > 1 ? ts.full_tiles / tiles_n : (p.M + C::TB - 1) / C::TB;
        tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    }
    const int m_base = tm * C::TB, n_base = tn * C::TB;
    M2::DmaRows<false, false> d;
    d.a = M2::make_dma_interior<C>(p.a, (uint32_t)(p.M * p.lda), (int)p.lda, m_base * (int)p.lda + k0);
    d.b = M2::make_dma_interior<C>(p.b, (uint32_t)(p.N * p.ldb), (int)p.ldb, n_base * (int)p.ldb + k0);
    M2::AccTile<P> acc;
    M2::mainloop<P>(stage0, stage1, d, klen, acc);
    if (chunk >= 0) {
        // this chunk's int32 accumulators -> its slot (rows / columns in range)
        int32_t *slot = slots + ((int64_t)(blockIdx.x - ts.full_tiles)) * 65536;
        M2::for_each_quad<P>(acc, [&](int ml, int nl, const v4i &v) {
            if (m_base + ml < p.M && n_base + nl < p.N) *reinterpret_cast<v4i *>(slot + ml * 256 + nl) = v;
        });
        return;
    }
    const bool full = m_base + C::TB <= p.M && n_base + C::TB <= p.N;
    if constexpr (EPI == EPI_W8A8_BF16 && VecOut) {
        if (full || p.N % 8 == 0) {
            // Scales fetched once per lane, output staged in LDS (free after the
            // mainloop's last barrier) and written as full rows; in an edge tile
            // (N % 8 == 0 there) rows past M and 8-column units past N are skipped.
            const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
            const int wrow = m_base + (wave / C::WAVES_N) * C::WM;
            const int wcol = n_base + (wave % C::WAVES_N) * C::WN;
            float sam[P::TI], none[P::TI];
            v4f swv[P::TJ];
#pragma unroll
            for (int i = 0; i < P::TI; ++i) sam[i] = p.sa[min(wrow + i * 16 + (lane & 15), p.M - 1)];
#pragma unroll
            for (int j = 0; j < P::TJ; ++j) {
                const int col = wcol + j * 16 + (lane >> 4) * 4;
                swv[j] = col < p.N ? *reinterpret_cast<const v4f *>(p.sw + col) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
            }
            int8_t *scratch = (wave < C::WAVES / 2 ? stage0 : stage1) + (wave % (C::WAVES / 2)) * (C::WM * C::WN * 2);
            M2::store_w8a8_bf16_staged<P, false>(
                acc, scratch, sam, none, swv,
                [&](int r) {
                    return wrow + r < p.M ? static_cast<uint16_t *>(p.d) + (int64_t)(wrow + r) * p.ldd + wcol : nullptr;
                },
                min(C::WN, p.N - wcol));
            return;
        }
    }
    if constexpr ((EPI == EPI_I32 || EPI == EPI_W8A8_F32) && VecOut) {
        if (p.ldd % 4 == 0 && (reinterpret_cast<uintptr_t>(p.d) & 15u) == 0 && (full || p.N % 4 == 0)) {
            // 32-bit rows staged in LDS (16 KiB per wave, two halves) and
            // written as 256-byte row segments instead of 16-byte quads.
            const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
            const int wrow = m_base + (wave / C::WAVES_N) * C::WM;
            const int wcol = n_base + (wave % C::WAVES_N) * C::WN;
            int8_t *scratch = (wave < C::WAVES / 2 ? stage0 : stage1) + (wave % (C::WAVES / 2)) * (C::WM / 2 * 256);
            auto row_dst = [&](int r) {
                return wrow + r < p.M ? static_cast<int32_t *>(p.d) + (int64_t)(wrow + r) * p.ldd + wcol : nullptr;
            };
            if constexpr (EPI == EPI_I32) {
                M2::store_x32x4_staged<P>(acc, scratch, [](int, int, const v4i &v) { return v; }, row_dst,
                                          min(C::WN, p.N - wcol));
            } else {
                // y = (sa[m] * sw[n]) * (float)acc, the scales fetched once per lane
                float sam[P::TI];
                v4f swv[P::TJ];
#pragma unroll
                for (int i = 0; i < P::TI; ++i) sam[i] = p.sa[min(wrow + i * 16 + (lane & 15), p.M - 1)];
#pragma unroll
                for (int j = 0; j < P::TJ; ++j) {
                    const int col = wcol + j * 16 + (lane >> 4) * 4;
                    swv[j] = col < p.N ? *reinterpret_cast<const v4f *>(p.sw + col) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
                }
                M2::store_x32x4_staged<P>(
                    acc, scratch,
                    [&](int r, int c, const v4i &v) {
                        const float sa_r = sam[r >> 4];
                        const v4f sw_c = swv[c >> 4];
                        return v4i{__float_as_int((sa_r * sw_c[0]) * (float)v[0]),
                                   __float_as_int((sa_r * sw_c[1]) * (float)v[1]),
                                   __float_as_int((sa_r * sw_c[2]) * (float)v[2]),
                                   __float_as_int((sa_r * sw_c[3]) * (float)v[3])};
                    },
                    row_dst, min(C::WN, p.N - wcol));
            }
            return;
        }
    }
    if constexpr (EPI == EPI_W8A8_F64 && VecOut) {
        if (p.ldd % 2 == 0 && (reinterpret_cast<uintptr_t>(p.d) & 15u) == 0 && (full || p.N % 4 == 0)) {
            // f64 rows staged in LDS (16 KiB per wave, four quarters) and
            // written as 512-byte row segments:
            // y = (double)(((float)sa[m] * (float)sw[n]) * (float)acc).
            const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
            const int wrow = m_base + (wave / C::WAVES_N) * C::WM;
            const int wcol = n_base + (wave % C::WAVES_N) * C::WN;
            int8_t *scratch = (wave < C::WAVES / 2 ? stage0 : stage1) + (wave % (C::WAVES / 2)) * (C::WM / 4 * 512);
            const double *sa64 = reinterpret_cast<const double *>(p.sa);
            const double *sw64 = reinterpret_cast<const double *>(p.sw);
            float sam[P::TI], swf[P::TJ][4];
#pragma unroll
            for (int i = 0; i < P::TI; ++i) sam[i] = (float)sa64[min(wrow + i * 16 + (lane & 15), p.M - 1)];
#pragma unroll
            for (int j = 0; j < P::TJ; ++j)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int col = wcol + j * 16 + (lane >> 4) * 4 + t;
                    swf[j][t] = col < p.N ? (float)sw64[col] : 0.0f;
                }
            auto bits = [](double x) { return (int64_t)__builtin_bit_cast(int64_t, x); };
            M2::store_x64x4_staged<P>(
                acc, scratch,
                [&](int r, int c, const v4i &v) {
                    const float sa_r = sam[r >> 4];
                    int64_t y[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) y[t] = bits((double)((sa_r * swf[c >> 4][t]) * (float)v[t]));
                    return M2::Quad64{v4i{(int)y[0], (int)(y[0] >> 32), (int)y[1], (int)(y[1] >> 32)},
                                      v4i{(int)y[2], (int)(y[2] >> 32), (int)y[3], (int)(y[3] >> 32)}};
                },
                [&](int r) {
                    return wrow + r < p.M ? static_cast<double *>(p.d) + (int64_t)(wrow + r) * p.ldd + wcol : nullptr;
                },
                min(C::WN, p.N - wcol));
            return;
        }
    }
    {
        const S8Epilogue<EPI, VecOut, ACT, BiasT> epi{p};
        if constexpr (EPI == EPI_S8 && VecOut) {
            if (p.ldd % 16 == 0 && (reinterpret_cast<uintptr_t>(p.d) & 15u) == 0 && (full || p.N % 16 == 0)) {
                store_s8_tile_staged<P>(acc, stage0, stage1, p, m_base, n_base, epi);
                return;
            }
        }
        M2::for_each_quad<P>(acc, [&](int ml, int nl, const v4i &v) { epi(m_base + ml, n_base + nl, v); });
    }
}

// Tail tiles of a split launch: a tile's K-chunk slots added in chunk order
// (int32, exact), then the epilogue of the unsplit kernel's general path.
// Workgroup (tail tile, 4 rows) x 64 column quads.
template <int EPI, bool VecOut, int ACT = ACT_NONE, typename BiasT = float>
__global__ __launch_bounds__(256) void gemm_s8_tail_reduce_kernel(S8Args p, TailSplit ts,
                                                                   const int32_t *__restrict__ slots) {
    const int tiles_n = (p.N + 255) / 256;
    const int ti = blockIdx.x;
    const int tm = ts.full_tiles / tiles_n + ti / tiles_n, tn = ti % tiles_n;
    const int row = blockIdx.y * 4 + (threadIdx.x >> 6), q = threadIdx.x & 63;
    const int m = tm * 256 + row, n0 = tn * 256 + 4 * q;
    if (m >= p.M || n0 >= p.N) return;
    const int32_t *s = slots + (int64_t)ti * ts.split * 65536 + row * 256 + 4 * q;
    v4i acc = *reinterpret_cast<const v4i *>(s);
    for (int c = 1; c < ts.split; ++c) {
        const v4i v = *reinterpret_cast<const v4i *>(s + (int64_t)c * 65536);
        acc = v4i{(int)((uint32_t)acc[0] + (uint32_t)v[0]), (int)((uint32_t)acc[1] + (uint32_t)v[1]),
                  (int)((uint32_t)acc[2] + (uint32_t)v[2]), (int)((uint32_t)acc[3] + (uint32_t)v[3])};
    }
    const S8Epilogue<EPI, VecOut, ACT, BiasT> epi{p};
    epi(m, n0, acc);
}

// The last M - m0 (<= kRowsPathMax) rows of an RCR GEMM whose other rows
// run as whole 256-row tiles (K % 128 == 0, 16-byte aligned rows, N % 16 ==
// 0).  A 256-row tile for them would stream its whole B panel at the pace of
// a full tile; here one workgroup of 8 waves owns 16 output columns, the
// waves split K into 8 contiguous runs of 64-byte chunks and stream their
// 16 B rows and the (at most 16 RF) A rows straight from global memory, U
// chunks in flight per batch, one v_mfma_i32_16x16x64_i8 per chunk and
// 16-row fragment of A (B first, A second, both taking k = 64 c + 16
// (lane / 16) + byte, so lane l ends with row m0 + 16 f + l % 16 and columns
// 4 (l / 16) .. + 3 of its 16).  The eight partial sums are added in LDS
// (int32 wrap-around, so the order does not matter) and go through the
// tiles' epilogue.
template <int EPI, bool VecOut, int ACT, typename BiasT, int RF>
__global__ __launch_bounds__(512) void gemm_s8_rcr_rows_kernel(S8Args p, int m0) {
    constexpr int U = RF == 1 ? 8 : RF <= 4 ? 4 : 2, WAVES = 8;
    __shared__ v4i part[WAVES][RF][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int8_t *arow[RF];
#pragma unroll
    for (int f = 0; f < RF; ++f) arow[f] = p.a + (int64_t)min(m0 + 16 * f + r16, p.M - 1) * p.lda + g * 16;
    const int8_t *brow = p.b + (int64_t)(n0 + r16) * p.ldb + g * 16;
    const int chunks = p.K >> 6;
    v4i acc[RF];
#pragma unroll
    for (int f = 0; f < RF; ++f) acc[f] = v4i{0, 0, 0, 0};
    // Wave w takes the contiguous chunks [c0, c1): 64 * (c1 - c0) bytes of
    // each of its 16 B rows in one span.
    const int c1 = (wave + 1) * chunks / WAVES;
    int c = wave * chunks / WAVES;
    for (; c + U <= c1; c += U) {
        v4i bv[U], av[U][RF];
#pragma unroll
        for (int u = 0; u < U; ++u)
            bv[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(brow + (int64_t)(c + u) * 64));
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int f = 0; f < RF; ++f) av[u][f] = *reinterpret_cast<const v4i *>(arow[f] + (int64_t)(c + u) * 64);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int f = 0; f < RF; ++f) acc[f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bv[u], av[u][f], acc[f], 0, 0, 0);
    }
    for (; c < c1; ++c) {
        const v4i bv = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(brow + (int64_t)c * 64));
#pragma unroll
        for (int f = 0; f < RF; ++f) {
            const v4i av = *reinterpret_cast<const v4i *>(arow[f] + (int64_t)c * 64);
            acc[f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bv, av, acc[f], 0, 0, 0);
        }
    }
#pragma unroll
    for (int f = 0; f < RF; ++f) part[wave][f][lane] = acc[f];
    __syncthreads();
    // wave w < RF adds up fragment w over the 8 waves
    if (wave >= RF) return;
    v4i sum = part[0][wave][lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
        const v4i v = part[w][wave][lane];
        sum = v4i{(int)((uint32_t)sum[0] + (uint32_t)v[0]), (int)((uint32_t)sum[1] + (uint32_t)v[1]),
                  (int)((uint32_t)sum[2] + (uint32_t)v[2]), (int)((uint32_t)sum[3] + (uint32_t)v[3])};
    }
    const S8Epilogue<EPI, VecOut, ACT, BiasT> epi{p};
    epi(m0 + 16 * wave + r16, n0 + 4 * g, sum);   // rows past M are not stored
}

template <bool VecOut, int ACT, typename BiasT>
struct U8Epilogue;
// Zero row / column sums for U8Epilogue when the correction is already in
// the accumulator.
__device__ const int kZeroSums[16] = {0};

// One last row (M = 1 decode steps; K % (1024 BT) == 0): a workgroup of 4
// waves owns 4 output columns and wave w streams B row n0 + w over all of K,
// 16 bytes per lane of every kilobyte straight into registers (BT kilobytes
// requested before their dot products), beside the same 16 bytes of the A
// row (an L2 hit); v_dot4_i32_i8 sums the products exactly in int32 (wrapping
// like the MFMA), a wave butterfly and LDS gather the 4 column sums and
// lane 0 of wave 0 runs the tiles' epilogue.  No LDS staging and 4096 waves
// at N = 4096: M = 1, N = K = 4096 over 20 rotated weight sets 4.84-4.96 us
// against 5.47-5.49 for gemm_s8_rcr_rows_dma_kernel (bit-identical), and
// 4.73 us for the same loads without the arithmetic.  From 2 rows on the A
// loads and dot products cost more than the layout saves (M = 2 / 4 / 8:
// 5.48 / 6.59 / 10.9 us against 5.52 / 5.66 / 5.98).
// U8: u8 operands (the u8 RCR SKUs): v_dot4_u32_u8 sums the products exactly
// (mod 2^32, no flip), and U8Epilogue runs with zero sums and no correction.
template <int EPI, bool VecOut, int ACT, typename BiasT, int BT, bool U8 = false>
__global__ __launch_bounds__(256) void gemm_s8_rcr_row1_kernel(S8Args p, int m0) {
    __shared__ int colsum[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * 4;
    const int nch = p.K >> 10;
    const int8_t *brow = p.b + (int64_t)(n0 + wave) * p.ldb + lane * 16;
    const int8_t *arow = p.a + (int64_t)m0 * p.lda + lane * 16;
    int acc = 0;
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
            for (int q = 0; q < 4; ++q) {
                if constexpr (U8)
                    acc = (int)__builtin_amdgcn_udot4((uint32_t)av[u][q], (uint32_t)bv[u][q], (uint32_t)acc, false);
                else
                    acc = __builtin_amdgcn_sdot4(av[u][q], bv[u][q], acc, false);
            }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc = (int)((uint32_t)acc + (uint32_t)__shfl_xor(acc, off, 64));
    if (lane == 0) colsum[wave] = acc;
    __syncthreads();
    if (threadIdx.x != 0) return;
    if constexpr (U8) {
        const U8Epilogue<VecOut, ACT, BiasT> epi{p, kZeroSums, kZeroSums, 0u};
        epi(0, 0, v4i{colsum[0], colsum[1], colsum[2], colsum[3]}, m0, n0);
    } else {
        const S8Epilogue<EPI, VecOut, ACT, BiasT> epi{p};
        epi(m0, n0, v4i{colsum[0], colsum[1], colsum[2], colsum[3]});
    }
}

// The last rows (at most 16 * RF), B streamed through LDS: K % 1024 == 0,
// K <= kRowsDmaMaxK, B 16-byte aligned with N * ldb < 2^31, dynamic LDS of
// max(16 * K, 16 KiB * RF) bytes.  A workgroup of 16 waves owns 16 output
// columns: wave w LDS-DMAs B row n0 + w whole, 1 KiB per instruction (every
// load a contiguous kilobyte of W, the GEMV's pattern, which streams HBM
// about 1.4x faster than 64-byte pieces of 16 rows), all of it issued before
// anything waits.  16-byte unit u of row r sits at slot u ^ r of the row,
// so the 16 rows of a fragment read fall in distinct banks; the swizzle
// stays inside each kilobyte, so every DMA instruction still fetches one
// contiguous kilobyte.  After one barrier wave w multiplies its contiguous
// K/16 bytes: B fragments from LDS, the RF 16-row A fragments of those
// bytes from global memory (issued before the barrier), one
// v_mfma_i32_16x16x64_i8 per 64 bytes and fragment with the operand roles
// of gemm_s8_rcr_rows_kernel, so lane l ends with row 16 f + l % 16 and
// columns 4 (l / 16) .. + 3.  The 16 partial sums go through LDS (int32
// wrap-around, order-free) and the tiles' epilogue.
constexpr int kRowsDmaMaxK = 8192;
// Up to this many last rows take gemm_s8_rcr_rows_dma_kernel (N = K = 4096,
// rotated weights: M = 1 / 16 in 5.45 / 6.8 us against 6.7 / 7.9 for
// gemm_s8_rcr_rows_kernel, and against 6.2 / 6.6 us for the staged kernel
// below with 1 KiB stages three deep).  From 17 rows on the staged kernel
// is faster: M = 17 / 24 / 32 in 6.96 / 7.05 / 7.18 us against 7.4 / 7.9 /
// 8.6 for this kernel with two fragments.
constexpr int kRowsDmaMaxRows = 16;
constexpr int kRowsDmaWaves = 16;

template <int EPI, bool VecOut, int ACT, typename BiasT, int RF>
__global__ __launch_bounds__(1024) void gemm_s8_rcr_rows_dma_kernel(S8Args p, int m0) {
    constexpr int WAVES = kRowsDmaWaves;
    constexpr int U = 4;                          // 64-byte chunks per batch of A loads
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];   // max(16 * K, 16 KiB * RF) bytes
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int mb = m0;                            // first of the last rows
    // B row n0 + wave, K bytes, into LDS row `wave` (K bytes per row).
    {
        const v4i rsrc = mfma2::make_rsrc(p.b, (uint32_t)((int64_t)p.N * p.ldb));
        const int voff = (n0 + wave) * (int)p.ldb + 16 * (lane ^ wave);
        int8_t *dst = lds + wave * p.K;
        for (int i = 0; i < p.K / 1024; ++i)
            mfma2::dma16(rsrc, voff, __builtin_amdgcn_readfirstlane(i * 1024), dst + i * 1024);
    }
    const int8_t *arow[RF];
#pragma unroll
    for (int f = 0; f < RF; ++f) arow[f] = p.a + (int64_t)min(mb + 16 * f + r16, p.M - 1) * p.lda + g * 16;
    const int span = p.K / WAVES;                 // bytes of K per wave, a multiple of 64
    const int kw = wave * span;
    v4i acc[RF];
#pragma unroll
    for (int f = 0; f < RF; ++f) acc[f] = v4i{0, 0, 0, 0};
    for (int c0 = 0; c0 < span; c0 += 64 * U) {
        v4i av[U][RF];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int f = 0; f < RF; ++f)
                av[u][f] = c0 + 64 * u < span ? *reinterpret_cast<const v4i *>(arow[f] + kw + c0 + 64 * u)
                                              : v4i{0, 0, 0, 0};
        if (c0 == 0) {
            // every DMA of the workgroup has landed (the A loads above were
            // issued after this wave's DMAs; vmcnt counts in order)
            mfma2::wait_dma();
            __syncthreads();
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + 64 * u >= span) break;
            const int unit = (kw + c0 + 64 * u) / 16 + g;   // 16-byte unit of row r16
            const v4i bv = *reinterpret_cast<const v4i *>(lds + r16 * p.K + 16 * (unit ^ r16));
#pragma unroll
            for (int f = 0; f < RF; ++f) acc[f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bv, av[u][f], acc[f], 0, 0, 0);
        }
    }
    __syncthreads();   // B no longer read: the partial sums reuse its LDS
    v4i *part = reinterpret_cast<v4i *>(lds);      // [WAVES][RF][64]
#pragma unroll
    for (int f = 0; f < RF; ++f) part[(wave * RF + f) * 64 + lane] = acc[f];
    __syncthreads();
    if (wave >= RF) return;
    v4i sum = part[wave * 64 + lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
        const v4i v = part[(w * RF + wave) * 64 + lane];
        sum = v4i{(int)((uint32_t)sum[0] + (uint32_t)v[0]), (int)((uint32_t)sum[1] + (uint32_t)v[1]),
                  (int)((uint32_t)sum[2] + (uint32_t)v[2]), (int)((uint32_t)sum[3] + (uint32_t)v[3])};
    }
    const S8Epilogue<EPI, VecOut, ACT, BiasT> epi{p};
    epi(mb + 16 * wave + r16, n0 + 4 * g, sum);   // rows past M are not stored
}

// The last rows, 17 to 16 RF of them, with A and B streamed through LDS in
// K stages of SB bytes, DEPTH stages in flight (K % SB == 0; A and B 16-byte
// aligned, (m0 + 16 RF) * lda and N * ldb below 2^31; dynamic LDS of
// DEPTH * (16 RF + 16) * SB bytes).  gemm_s8_rcr_rows_kernel reads its A
// fragments from global memory as 64-byte pieces of 16 rows, and every one
// of the N / 16 workgroups reads all of A: that pattern moves L2-resident
// bytes 2.5x slower than whole kilobytes (64 MB of A at M = 64: 8.1
// against 3.2 us) and dominated the pass.  Here a workgroup of 16 waves
// LDS-DMAs each K stage of its 16 RF A rows (rows past M land as zeros) and
// of its 16 B rows, 1024 / SB whole row pieces per instruction, all before
// anything waits.  16-byte unit u of row r of a stage sits at slot
// u ^ (r & 15), so fragment reads are conflict-free.  Wave w owns 64-byte
// chunk w % CH of every stage (CH = SB / 64) and row fragments
// w / CH + (16 / CH) i; its sums over the stages go through LDS (int32
// wrap-around: order-free) and waves 0 .. RF - 1 run the tiles' epilogue
// for fragment w.
// 512-byte stages, two in flight: at N = K = 4096 (M = 33 / 64 / 100 / 128)
// 8.0 / 8.8 / 11.3 / 11.6 us, against 9.8-10.3 / 10.0-10.5 / 12.0-13.2 /
// 12.3-13.5 us for 256-byte stages two to four deep; three 512-byte stages
// measure the same as two (kRowsStagedSB, kRowsStagedDepth).

// U8: u8 x u8 operands (RCR u8 SKUs; EPI unused) through the signed MFMA:
// fragments flipped to u - 128 and the correction of
// sum(u_a u_b) = acc_s + 128 (sum a' + sum b') + 16384 K folded into the same
// accumulator: 64 * sum a' and 64 * sum b' are two MFMAs each against a
// fragment of bytes 64 (int32 wrap-around, exact mod 2^32), 16384 K in the
// epilogue.
//
// RowB: B row-major [K, N] (the RRR SKUs): a stage's B region holds its SB
// k-rows of the 16 NB columns as they lie in memory (row pitch 16 NB bytes,
// whole-row DMAs, the K position moving the row by k0 * ldb), and the B
// fragments are rebuilt with ds_read_b64_tr_b8 as in PolicyI8RowB: the lane
// pair (2j, 2j + 1) of a 16-lane group points at k-row j, lane i gets 8
// consecutive k of column i.
template <int EPI, bool VecOut, int ACT, typename BiasT, int RF, int NB, int SB, int DEPTH, bool U8 = false,
          bool RowB = false>
__global__ __launch_bounds__(1024) void gemm_s8_rcr_rows_staged_kernel(S8Args p, int m_first) {
    // blockIdx.y: 16 RF-row block of the pass (several when the pass covers
    // more rows than one workgroup holds)
    const int m0 = m_first + blockIdx.y * 16 * RF;
    constexpr int WAVES = 16, CH = SB / 64;                  // 64-byte chunks per stage
    // With fewer (fragment, chunk) pairs than waves (RF * CH < 16) the first
    // RF * CH waves hold one each and the others only DMA.
    constexpr bool ALL = RF * CH >= WAVES;
    constexpr int FPW = ALL ? RF * CH / WAVES : 1;            // A row fragments per wave
    constexpr int FSTEP = WAVES / CH;
    constexpr int ROWS = 16 * RF + 16 * NB;                   // A then B rows of a stage
    constexpr int STAGE = ROWS * SB;                          // bytes
    constexpr int UPR = SB / 16;                              // 16-byte units per row
    constexpr int NI = ROWS * UPR / 64;                       // 1 KiB DMA instructions per stage
    constexpr int HI = (NI + WAVES - 1) / WAVES, LO = NI / WAVES;
    static_assert((!ALL || RF * CH % WAVES == 0) && UPR >= 16 && (ROWS * UPR) % 64 == 0 && DEPTH >= 2 &&
                      DEPTH <= 4 && RF * NB * CH * 1024 <= 160 * 1024 && DEPTH * STAGE <= 160 * 1024,
                  "stage split");
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
    // this wave's DMA instructions j = wave, wave + 16, ...: units 64 j ..
    // 64 j + 63 of the row-major stage (A rows first), lane L fetching unit
    // (64 j + L) % UPR of row (64 j + L) / UPR
    auto dma_stage = [&](int st, int8_t *buf) {
        const int k0 = st * SB;
        for (int j = wave; j < NI; j += WAVES) {
            const int idx = 64 * j + lane;
            const int r = idx / UPR, slot = idx % UPR;
            const int unit = slot ^ (r & 15);
            if (r < 16 * RF) {
                mfma2::dma16(ra, (int)((int64_t)(m0 + r) * p.lda) + 16 * unit, k0, buf + j * 1024);
            } else if constexpr (RowB) {
                // unit ib of the B region: k-row ib / NB, 16 columns ib % NB
                const int ib = idx - 16 * RF * UPR;
                mfma2::dma16(rb, (ib / NB) * (int)p.ldb + n0 + 16 * (ib % NB),
                             __builtin_amdgcn_readfirstlane(k0 * (int)p.ldb), buf + j * 1024);
            } else {
                mfma2::dma16(rb, (int)((int64_t)(n0 + r - 16 * RF) * p.ldb) + 16 * unit, k0, buf + j * 1024);
            }
        }
    };
    // waves below NI % 16 issue HI instructions per stage, the others LO
    const bool hi = NI % WAVES == 0 || wave < NI % WAVES;
    const int ns = p.K / SB;
    for (int st = 0; st < DEPTH && st < ns; ++st) dma_stage(st, lds + st * STAGE);
    const int c = wave % CH, f0 = wave / CH;
    const bool active = ALL || wave < RF * CH;   // wave-uniform
    v4i acc[FPW][NB];
#pragma unroll
    for (int i = 0; i < FPW; ++i)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[i][nb] = v4i{0, 0, 0, 0};
    const int sl = 16 * ((4 * c + g) ^ r16);                     // row & 15 == r16 for every fragment row
    for (int st = 0; st < ns; ++st) {
        // stage st has landed once at most the later stages' DMAs are outstanding
        const int later = min(DEPTH - 1, ns - 1 - st);
        if (later == 0) mfma2::wait_vmcnt<0>();
        else if (later == 1) { if (hi) mfma2::wait_vmcnt<HI>(); else mfma2::wait_vmcnt<LO>(); }
        else if (later == 2) { if (hi) mfma2::wait_vmcnt<2 * HI>(); else mfma2::wait_vmcnt<2 * LO>(); }
        else { if (hi) mfma2::wait_vmcnt<3 * HI>(); else mfma2::wait_vmcnt<3 * LO>(); }
        __syncthreads();
        int8_t *buf = lds + (st % DEPTH) * STAGE;
        if (active) {
        v4i bv[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if constexpr (RowB) {
                const int kb = 64 * c + 16 * g + (r16 >> 1);
                const int8_t *q = buf + 16 * RF * SB + kb * (16 * NB) + 16 * nb + ((lane & 1) << 3);
                const mfma2::v2i_t lo = mfma2::ds_read_tr8(q), hi = mfma2::ds_read_tr8(q + 8 * 16 * NB);
                bv[nb] = v4i{lo[0], lo[1], hi[0], hi[1]};
            } else {
                bv[nb] = *reinterpret_cast<const v4i *>(buf + (16 * RF + 16 * nb + r16) * SB + sl);
            }
            if constexpr (U8) bv[nb] = u8_flip(bv[nb]);
        }
        constexpr v4i c64 = {0x40404040, 0x40404040, 0x40404040, 0x40404040};
#pragma unroll
        for (int i = 0; i < FPW; ++i) {
            v4i av = *reinterpret_cast<const v4i *>(buf + (16 * (f0 + FSTEP * i) + r16) * SB + sl);
            if constexpr (U8) av = u8_flip(av);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                acc[i][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bv[nb], av, acc[i][nb], 0, 0, 0);
                if constexpr (U8) {
                    acc[i][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c64, av, acc[i][nb], 0, 0, 0);
                    acc[i][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c64, av, acc[i][nb], 0, 0, 0);
                    acc[i][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bv[nb], c64, acc[i][nb], 0, 0, 0);
                    acc[i][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bv[nb], c64, acc[i][nb], 0, 0, 0);
                }
            }
        }
        }
        __syncthreads();   // every wave is done with this buffer
        if (st + DEPTH < ns) dma_stage(st + DEPTH, buf);
    }
    // partial sums of (A fragment f, B fragment nb), chunk c: part[f][nb][c][lane]
    v4i *part = reinterpret_cast<v4i *>(lds);
    if (active) {
#pragma unroll
        for (int i = 0; i < FPW; ++i)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) part[(((f0 + FSTEP * i) * NB + nb) * CH + c) * 64 + lane] = acc[i][nb];
    }
    __syncthreads();
    const S8Epilogue<EPI, VecOut, ACT, BiasT> epi{p};
    // u8: au = acc - kcorr with zero sums, kcorr = -16384 K (mod 2^32)
    const U8Epilogue<VecOut, ACT, BiasT> epi_u8{p, kZeroSums, kZeroSums, 0u - 16384u * (uint32_t)p.K};
    for (int e = wave; e < RF * NB; e += WAVES) {
        const int f = e % RF, nb = e / RF;
        v4i sum = part[((f * NB + nb) * CH) * 64 + lane];
#pragma unroll
        for (int cc = 1; cc < CH; ++cc) {
            const v4i v = part[((f * NB + nb) * CH + cc) * 64 + lane];
            sum = v4i{(int)((uint32_t)sum[0] + (uint32_t)v[0]), (int)((uint32_t)sum[1] + (uint32_t)v[1]),
                      (int)((uint32_t)sum[2] + (uint32_t)v[2]), (int)((uint32_t)sum[3] + (uint32_t)v[3])};
        }
        if constexpr (U8) epi_u8(r16, 4 * g, sum, m0 + 16 * f, n0 + 16 * nb);   // rows past M are not stored
        else epi(m0 + 16 * f + r16, n0 + 16 * nb + 4 * g, sum);
    }
}

// RRR fast path: A through the interior DMA, row-major B through the
// transposing fragment reads (PolicyI8RowB); same tiles and epilogue as RCR.
template <bool VecOut, int ACT, typename BiasT>
__global__ __launch_bounds__(DmaCfg::NT, 1) void gemm_s8_rrr_dma_kernel(S8Args p) {
    namespace M2 = mfma2;
    typedef M2::PolicyI8RowB<DmaCfg> P;
    __shared__ __attribute__((aligned(1024))) int8_t stage0[2 * M2::OPER];
    __shared__ __attribute__((aligned(1024))) int8_t stage1[2 * M2::OPER];
    // Edge tiles: A rows past M load as zeros (past the buffer's byte count);
    // B columns past N read bytes of the next k-row (or zeros after the
    // last), which only reach output columns that are not stored.
    const int tiles_m = (p.M + M2::BM - 1) / M2::BM, tiles_n = (p.N + M2::BN - 1) / M2::BN;
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m_base = tm * M2::BM, n_base = tn * M2::BN;
    M2::DmaRowsRrr d;
    d.a = M2::make_dma_interior<DmaCfg>(p.a, (uint32_t)(p.M * p.lda), (int)p.lda, m_base * (int)p.lda);
    d.b = M2::make_dma_row_b<DmaCfg>(p.b, (uint32_t)(p.K * p.ldb), (int)p.ldb, n_base);
    M2::AccTile<P> acc;
    M2::mainloop<P>(stage0, stage1, d, p.K, acc);
    const S8Epilogue<EPI_S8, VecOut, ACT, BiasT> epi{p};
    const bool full = m_base + M2::BM <= p.M && n_base + M2::BN <= p.N;
    if constexpr (VecOut) {
        if (p.ldd % 16 == 0 && (reinterpret_cast<uintptr_t>(p.d) & 15u) == 0 && (full || p.N % 16 == 0)) {
            store_s8_tile_staged<P>(acc, stage0, stage1, p, m_base, n_base, epi);
            return;
        }
    }
    M2::for_each_quad<P>(acc, [&](int ml, int nl, const v4i &v) { epi(m_base + ml, n_base + nl, v); });
}

// ---- u8 x u8 RRR (B row-major [K,N]) ----------------------------------------
// Operands run through the signed MFMA as s = u - 128; with the raw-byte sums
// of each A row and B column the unsigned accumulator is restored exactly
// modulo 2^32:  sum_k u_a*u_b = acc_s + 128*(rowsum + colsum) - 16384*K_pad,
// K_pad = the k extent of the stages run (zero-padded k are 0 in the sums and
// (-128)*(-128) in acc_s).
// D = sat_u8(rne(act(alpha*acc + beta*C [+ bias[n]]))) (gemm_u8_rrr_sm80 /
// ..._bias semantics, baracuda_int8_rrr_sm80.cuh).
template <bool VecOut, int ACT, typename BiasT>
struct U8Epilogue {
    const S8Args &p;
    const int *rs;        // [256] tile row sums of A
    const int *cs;        // [256] tile column sums of B
    uint32_t kcorr;       // 16384 * K_pad (mod 2^32), subtracted
    // Whole group of 4 columns (N % 4 == 0): the 4 result bytes.
    // HasC: beta != 0 and C given; CVec: the 4 C bytes read as one dword
    // (ldc and C 4-byte aligned) -- both decided once per tile by the caller.
    template <bool HasC, bool CVec = false>
    __device__ __forceinline__ uint32_t pack_u8(int ml, int nl, const v4i &v, int m_base, int n_base) const {
        const int m = m_base + ml, n0 = n_base + nl;
        const uint32_t rsum = (uint32_t)rs[ml];
        const uint8_t *c = reinterpret_cast<const uint8_t *>(p.c);
        uint32_t c4 = 0;
        if constexpr (HasC && CVec) c4 = *reinterpret_cast<const uint32_t *>(c + (int64_t)m * p.ldc + n0);
        uint32_t w = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t au = (uint32_t)v[r] + 128u * (rsum + (uint32_t)cs[nl + r]) - kcorr;
            float z = p.alpha * (float)(int32_t)au;
            if constexpr (HasC)
                z += p.beta * (float)(CVec ? (uint8_t)(c4 >> (8 * r)) : c[(int64_t)m * p.ldc + n0 + r]);
            if constexpr (ACT != ACT_NONE) {
                z += (float)static_cast<const BiasT *>(p.bias)[n0 + r];
                z = activation<ACT>(z);
            }
            w |= (uint32_t)sat_cast_u8(z) << (8 * r);
        }
        return w;
    }
    __device__ __forceinline__ void operator()(int ml, int nl, const v4i &v, int m_base,
                                               int n_base) const {
        const int m = m_base + ml, n0 = n_base + nl;
        if (m >= p.M || n0 >= p.N) return;
        const int count = VecOut ? 4 : (p.N - n0 < 4 ? p.N - n0 : 4);
        const uint32_t rsum = (uint32_t)rs[ml];
        uint8_t *d = static_cast<uint8_t *>(p.d) + (int64_t)m * p.ldd + n0;
        const uint8_t *c = reinterpret_cast<const uint8_t *>(p.c);
        uint8_t o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t au = (uint32_t)v[r] + 128u * (rsum + (uint32_t)cs[nl + r]) - kcorr;
            float z = p.alpha * (float)(int32_t)au;
            if (p.beta != 0.0f && c != nullptr && r < count)
                z += p.beta * (float)c[(int64_t)m * p.ldc + n0 + r];
            if constexpr (ACT != ACT_NONE) {
                if (r < count) z += (float)static_cast<const BiasT *>(p.bias)[n0 + r];
                z = activation<ACT>(z);
            }
            o[r] = sat_cast_u8(z);
        }
        if constexpr (VecOut) {
            *reinterpret_cast<uint32_t *>(d) = (uint32_t)o[0] | ((uint32_t)o[1] << 8) |
                                               ((uint32_t)o[2] << 16) | ((uint32_t)o[3] << 24);
        } else {
            for (int r = 0; r < count; ++r) d[r] = o[r];
        }
    }
};

// Row sums of a [256][*] tile slice: lanes 2r, 2r+1 of wave w hold halves of
// row 32w + r.  Writes dst[32w + r].
__device__ __forceinline__ void park_row_sums(uint32_t v, int *dst) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v += __shfl_xor(v, 1, 64);
    if ((lane & 1) == 0) dst[32 * wave + (lane >> 1)] = (int)v;
}

// u8 outputs of a whole tile: staged 16-byte row stores when D allows them.
template <bool VecOut, class P, class Epi>
__device__ __forceinline__ void store_u8_tile(const mfma2::AccTile<P> &acc, int8_t *stage0, int8_t *stage1,
                                              const S8Args &p, int m_base, int n_base, const Epi &epi) {
    if constexpr (VecOut) {
        if (p.ldd % 16 == 0 && (reinterpret_cast<uintptr_t>(p.d) & 15u) == 0) {
            const int wave = threadIdx.x >> 6;
            const int wrow = (wave / DmaCfg::WAVES_N) * DmaCfg::WM;
            const int wcol = (wave % DmaCfg::WAVES_N) * DmaCfg::WN;
            int8_t *scratch = (wave < 4 ? stage0 : stage1) + (wave & 3) * (DmaCfg::WM * DmaCfg::WN);
            auto staged = [&](auto has_c, auto c_vec) {
                mfma2::store_u8x4_staged<P>(
                    acc, scratch,
                    [&](int r, int c, const v4i &v) {
                        return epi.template pack_u8<decltype(has_c)::value, decltype(c_vec)::value>(
                            wrow + r, wcol + c, v, m_base, n_base);
                    },
                    [&](int r) {
                        return static_cast<int8_t *>(p.d) + (int64_t)(m_base + wrow + r) * p.ldd + n_base + wcol;
                    });
            };
            // the C term decided once per tile, not per element
            if (p.beta != 0.0f && p.c != nullptr) {
                if (p.ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(p.c) & 3u) == 0)
                    staged(std::true_type{}, std::true_type{});
                else
                    staged(std::true_type{}, std::false_type{});
            } else {
                staged(std::false_type{}, std::false_type{});
            }
            return;
        }
    }
    mfma2::for_each_quad<P>(acc, [&](int ml, int nl, const v4i &v) { epi(ml, nl, v, m_base, n_base); });
}

template <bool VecOut, int ACT, typename BiasT>
__global__ __launch_bounds__(DmaCfg::NT, 1) void gemm_u8_rrr_dma_kernel(S8Args p) {
    namespace M2 = mfma2;
    typedef M2::PolicyU8RowB<DmaCfg> P;
    __shared__ __attribute__((aligned(1024))) int8_t stage0[2 * M2::OPER];
    __shared__ __attribute__((aligned(1024))) int8_t stage1[2 * M2::OPER];
    const int tiles_m = p.M / M2::BM, tiles_n = p.N / M2::BN;
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m_base = tm * M2::BM, n_base = tn * M2::BN;
    M2::DmaRowsRrr d;
    d.a = M2::make_dma_interior<DmaCfg>(p.a, (uint32_t)(p.M * p.lda), (int)p.lda, m_base * (int)p.lda);
    d.b = M2::make_dma_row_b<DmaCfg>(p.b, (uint32_t)(p.K * p.ldb), (int)p.ldb, n_base);
    M2::AccTile<P> acc;
    typename P::Sums sums;
    sums.ra = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) sums.cb[q] = 0;
    M2::mainloop<P>(stage0, stage1, d, p.K, acc, sums);
    // Park: row sums directly; column partials per wave in [8][256], then
    // summed; above the staged-store scratch of waves 4..7 (stage1's first 32 KiB).
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int *sc = reinterpret_cast<int *>(stage1 + 40 * 1024);   // rs[256] | cs[256] | part[8][256]
    park_row_sums(sums.ra, sc);
    // Lane i of group g holds column 16*(g + 4q) + i over this wave's 16 k-rows
    // in cb[q]: every column exactly once per wave.
#pragma unroll
    for (int q = 0; q < 4; ++q) sc[512 + 256 * wave + 16 * ((lane >> 4) + 4 * q) + (lane & 15)] = (int)sums.cb[q];
    __syncthreads();
    if (threadIdx.x < 256) {
        int t = 0;
#pragma unroll
        for (int w = 0; w < 8; ++w) t += sc[512 + 256 * w + threadIdx.x];
        sc[256 + threadIdx.x] = t;
    }
    __syncthreads();
    const U8Epilogue<VecOut, ACT, BiasT> epi{p, sc, sc + 256, 16384u * (uint32_t)p.K};
    store_u8_tile<VecOut, P>(acc, stage0, stage1, p, m_base, n_base, epi);
}

// ---- u8 pre-pass (when the caller gives a workspace) ------------------------
// Writes the operands flipped to u - 128 (so the GEMM is the plain s8 RRR
// loop) and their exact int32 sums: rowsum[m] = sum_k A[m, k], colsum[n] =
// sum_k B[k, n] (K < 2^23).  The A pass (one wave per row, udot4 over
// 16-byte chunks) also zeroes colsum; the B pass adds K-slices of 4-column
// groups with integer atomics (exact, so the order does not matter).
__global__ __launch_bounds__(256) void u8_prep_a_kernel(const uint8_t *__restrict__ a, int64_t lda, int M, int K,
                                                        int8_t *__restrict__ af, int *__restrict__ rowsum,
                                                        int *__restrict__ colsum, int N) {
    const int gid = blockIdx.x * 256 + threadIdx.x;
    if (gid < N) colsum[gid] = 0;
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    const uint8_t *row = a + (int64_t)m * lda;
    int8_t *frow = af + (int64_t)m * K;
    uint32_t acc = 0;
    for (int c = lane; c < (K >> 4); c += 64) {
        const v4i w = *reinterpret_cast<const v4i *>(row + 16 * c);
        acc = u8_sum16(w, acc);
        *reinterpret_cast<v4i *>(frow + 16 * c) = u8_flip(w);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += (uint32_t)__shfl_xor((int)acc, off, 64);
    if (lane == 0) rowsum[m] = (int)acc;
}

constexpr int kU8ColSlice = 256;   // K rows per B-pass workgroup (16 per thread row lane)

// Workgroup: 256 columns x kU8ColSlice rows; thread (c, r) = (tid % 16,
// tid / 16) takes the 16-byte column chunk c of rows r, r + 16, ...; the 16
// row lanes are combined in LDS and each column gets one atomic.
__global__ __launch_bounds__(256) void u8_prep_b_kernel(const uint8_t *__restrict__ b, int64_t ldb, int K, int N,
                                                        int8_t *__restrict__ bf, int *__restrict__ colsum) {
    __shared__ int part[16][257];
    const int c = threadIdx.x & 15, r = threadIdx.x >> 4;
    const int n = blockIdx.x * 256 + 16 * c;
    const int k0 = blockIdx.y * kU8ColSlice, k1 = min(K, k0 + kU8ColSlice);
    // Two 16-bit lanes per accumulator word: 16 rows of 255 fit easily.
    uint32_t acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0;
    if (n < N) {
#pragma unroll 4
        for (int k = k0 + r; k < k1; k += 16) {
            const v4i w = *reinterpret_cast<const v4i *>(b + (int64_t)k * ldb + n);
            *reinterpret_cast<v4i *>(bf + (int64_t)k * N + n) = u8_flip(w);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[2 * q] += (uint32_t)w[q] & 0x00ff00ffu;
                acc[2 * q + 1] += ((uint32_t)w[q] >> 8) & 0x00ff00ffu;
            }
        }
    }
    // column 16c + 4q + {0, 2} in acc[2q] lanes {lo, hi}; {1, 3} in acc[2q + 1]
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        part[r][16 * c + 4 * q] = (int)(acc[2 * q] & 0xffffu);
        part[r][16 * c + 4 * q + 2] = (int)(acc[2 * q] >> 16);
        part[r][16 * c + 4 * q + 1] = (int)(acc[2 * q + 1] & 0xffffu);
        part[r][16 * c + 4 * q + 3] = (int)(acc[2 * q + 1] >> 16);
    }
    __syncthreads();
    const int col = blockIdx.x * 256 + threadIdx.x;
    if (col < N) {
        int t = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) t += part[i][threadIdx.x];
        atomicAdd(colsum + col, t);
    }
}

// The LDS-DMA s8 RRR GEMM on the flipped operands (p.a / p.b point at them)
// with the u8 epilogue over the pre-pass sums.
template <bool VecOut, int ACT, typename BiasT>
__global__ __launch_bounds__(DmaCfg::NT, 1) void gemm_u8_rrr_ws_kernel(S8Args p, const int *__restrict__ rowsum,
                                                                       const int *__restrict__ colsum) {
    namespace M2 = mfma2;
    typedef M2::PolicyI8RowB<DmaCfg> P;
    __shared__ __attribute__((aligned(1024))) int8_t stage0[2 * M2::OPER];
    __shared__ __attribute__((aligned(1024))) int8_t stage1[2 * M2::OPER];
    const int tiles_m = p.M / M2::BM, tiles_n = p.N / M2::BN;
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m_base = tm * M2::BM, n_base = tn * M2::BN;
    M2::DmaRowsRrr d;
    d.a = M2::make_dma_interior<DmaCfg>(p.a, (uint32_t)(p.M * p.lda), (int)p.lda, m_base * (int)p.lda);
    d.b = M2::make_dma_row_b<DmaCfg>(p.b, (uint32_t)(p.K * p.ldb), (int)p.ldb, n_base);
    M2::AccTile<P> acc;
    M2::mainloop<P>(stage0, stage1, d, p.K, acc);
    // The tile's 256 row and 256 column sums into LDS (free after the loop),
    // above the staged-store scratch of waves 4..7.
    static_assert(DmaCfg::NT == 512, "one sum per thread");
    int *sc = reinterpret_cast<int *>(stage1 + 40 * 1024);
    sc[threadIdx.x] = threadIdx.x < 256 ? rowsum[m_base + threadIdx.x] : colsum[n_base + threadIdx.x - 256];
    __syncthreads();
    const U8Epilogue<VecOut, ACT, BiasT> epi{p, sc, sc + 256, 16384u * (uint32_t)p.K};
    store_u8_tile<VecOut, P>(acc, stage0, stage1, p, m_base, n_base, epi);
}

// Workspace of the pre-pass path: sums (256-byte aligned), then A and B flipped.
inline size_t u8_ws_sums_bytes(int M, int N) { return ((size_t)(M + N) * 4 + 255) & ~(size_t)255; }
inline size_t u8_rrr_workspace_bytes(int M, int N, int K) {
    return u8_ws_sums_bytes(M, N) + (((size_t)M * K + 255) & ~(size_t)255) + (size_t)K * N;
}

template <bool Aligned, int ACT, typename BiasT>
__global__ __launch_bounds__(NT, 1) void gemm_u8_rrr_kernel(S8Args p) {
    __shared__ __attribute__((aligned(16))) int8_t lds[4 * LDS_TILE];
    const int tiles_m = (p.M + BM - 1) / BM;
    const int tiles_n = (p.N + BN - 1) / BN;
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m_base = tm * BM, n_base = tn * BN;
    const int tid = threadIdx.x;
    RowSet as;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int r = i * LOAD_ROWS + (tid >> 3);
        as.ptr[i] = p.a + (int64_t)min(m_base + r, p.M - 1) * p.lda;
    }
    v4i acc[TM][TN];
    U8Sums sums;
    mainloop_rrr<Elem::U8, !Aligned, !Aligned>(lds, as, p.b, p.ldb, p.N, n_base, p.K, acc, &sums);
    int *sc = reinterpret_cast<int *>(lds);
    park_row_sums(sums.ra, sc);
    park_row_sums(sums.cb, sc + 256);
    __syncthreads();
    const uint32_t kpad = (uint32_t)((p.K + BK - 1) / BK) * (uint32_t)BK;
    const U8Epilogue<false, ACT, BiasT> epi{p, sc, sc + 256, 16384u * kpad};
    for_each_fragment(acc, [&](int ml, int nl, const v4i &v) { epi(ml, nl, v, m_base, n_base); });
}

// Whole-tile problems the LDS-DMA u8 RRR kernels take.
inline bool u8_rrr_dma_eligible(const S8Args &p) {
    return p.K % mfma2::BK == 0 && p.M % mfma2::BM == 0 && p.N % mfma2::BN == 0 && p.lda % 16 == 0 &&
           p.ldb % 16 == 0 && aligned16(p.a) && aligned16(p.b) && (int64_t)p.M * p.lda < (1ll << 31) &&
           (int64_t)p.K * p.ldb < (1ll << 31);
}

// ... of which those whose operands the pre-pass can rewrite into a workspace.
inline bool u8_rrr_prepass_eligible(const S8Args &p) {
    return u8_rrr_dma_eligible(p) && (int64_t)p.K * p.N < (1ll << 31);
}

// u8 RRR last rows (decode-sized M; M % 256 in [1, 128] when a row of tiles
// would start another round): the staged last-rows kernel with both its u8
// and row-major-B flags, 64 columns per workgroup where N allows; main tiles
// above the rows on the LDS-DMA u8 RRR kernel.  False when the shape does
// not fit.  N = K = 4096, M = 1 / 16 on the general kernel: 87.4 / 86.6 us.
// Row blocks of a last-rows launch of the u8 RCR and s8 / u8 RRR SKUs
// (the int8 RCR launcher applies the same two rules inline): a small grid
// (`whole`: all M rows) as 64-row blocks when they fit one round of
// workgroups, else 128-row blocks; 33-128 last rows below N = 6144 as the
// row blocks of mfma2::last_rows_blocks; otherwise one block of the fewest
// fragments (1 / 2 / 4 / 8) that hold the rows.  rf: 16-row fragments per block.  K = 4096,
// graph replay, against one 128-row block (M = 100) or 128-row blocks
// (M = 200 / 256): N = 4096, M = 100 u8 RCR 14.7 -> 12.4, s8 RRR 13.8 ->
// 11.8, u8 RRR 18.3 -> 14.0 us; N = 2048, M = 100 / 256 u8 RCR 12.9 / 13.7
// -> 8.8 / 11.5, s8 RRR 12.8 / 13.8 -> 9.8 / 11.7, u8 RRR 16.7 / 17.7 ->
// 10.9 / 13.5 us; s8 RRR N = 4096, M = 200 / 256 14.3 / 15.0 -> 14.8 /
// 15.1 us (the one loss).
inline void rows_blocks_plan(int M, int N, int rem, bool whole, int &rf, int &blocks, int &nb) {
    if (whole) {
        const int b4 = (M + 63) / 64, n4 = mfma2::last_rows_col_frags(N, b4);
        if (b4 * (N / (16 * n4)) <= 256) {
            rf = 4;
            blocks = b4;
            nb = n4;
            return;
        }
        rf = 8;
        blocks = (M + 127) / 128;
        nb = mfma2::last_rows_col_frags(N, blocks);
        return;
    }
    nb = mfma2::last_rows_col_frags(N, 1);
    if (nb == 1 && rem > 32) {
        mfma2::last_rows_blocks(rem, N, rf, blocks, nb);
        return;
    }
    // up to 16 rows: one fragment, 8 of the 16 waves multiplying (K = 4096,
    // M = 1-16, against two fragments: N = 4096 u8 RCR 7.5 -> 6.6, s8 RRR
    // 9.2 -> 8.5, u8 RRR 9.8 -> 8.7 us; N = 14336 14.0 -> 12.1, 14.8 ->
    // 13.7, 17.5 -> 14.6 us)
    rf = rem <= 16 ? 1 : rem <= 32 ? 2 : (rem <= 64 ? 4 : 8);
    blocks = 1;
}

template <int ACT, typename BiasT>
bool launch_u8_rrr_rows(const S8Args &p, hipStream_t stream) {
    int rem = mfma2::last_rows_pass(p.M, p.N, 128), blocks = 1;
    bool whole = false;
    if (rem == 0 && (p.M <= 256 || (p.M <= 512 && p.M % 256 != 0)) && p.N % 16 == 0) {
        // a small grid of 256-row tiles: all rows as 128-row blocks of the
        // last-rows kernel.  N = K = 4096: M = 200 / 256 / 384 in 36.0 /
        // 35.7 / 35.9 us against 87 / 60 (pre-pass workspace) / 114.7; whole-
        // tile M = 512 stays on the tiles (60 us)
        rem = 128;
        blocks = (p.M + 127) / 128;
        whole = true;
    }
    if (rem == 0 || p.K % 512 != 0 || p.lda % 16 != 0 || p.ldb % 16 != 0 || !aligned16(p.a) || !aligned16(p.b) ||
        !dma_extent_ok(p.M, p.lda) || (int64_t)p.K * p.ldb + mfma2::BN >= (1ll << 31))
        return false;
    S8Args pm = p;
    pm.M = whole ? 0 : p.M - rem;
    if (pm.M > 0 && !u8_rrr_dma_eligible(pm)) return false;
    const bool vec = p.ldd % 4 == 0 && (reinterpret_cast<uintptr_t>(p.d) % 4) == 0;
    if (pm.M > 0) {
        const int tiles = (pm.M / mfma2::BM) * (p.N / mfma2::BN);
        if (vec)
            hipLaunchKernelGGL((gemm_u8_rrr_dma_kernel<true, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0, stream, pm);
        else
            hipLaunchKernelGGL((gemm_u8_rrr_dma_kernel<false, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0, stream, pm);
    }
    int rf, nb;   // as the s8 RRR pass
    rows_blocks_plan(p.M, p.N, rem, whole, rf, blocks, nb);
#define BK_U8RRRROWS(RF, NB, SB, DEPTH)                                                                        \
    if (rf == (RF) && nb == (NB)) {                                                                              \
        const size_t lds = std::max((size_t)(DEPTH) * (16 * (RF) + 16 * (NB)) * (SB), (size_t)(RF) * (NB) * ((SB) / 64) * 1024); \
        if (vec)                                                                                                \
            hipLaunchKernelGGL((gemm_s8_rcr_rows_staged_kernel<0, true, ACT, BiasT, RF, NB, SB, DEPTH, true, true>), \
                               dim3(p.N / (16 * (NB)), blocks), dim3(1024), lds, stream, p, pm.M);                      \
        else                                                                                                    \
            hipLaunchKernelGGL((gemm_s8_rcr_rows_staged_kernel<0, false, ACT, BiasT, RF, NB, SB, DEPTH, true, true>), \
                               dim3(p.N / (16 * (NB)), blocks), dim3(1024), lds, stream, p, pm.M);                      \
        return true;                                                                                            \
    }
    BK_U8RRRROWS(1, 1, 512, 3)
    BK_U8RRRROWS(1, 2, 512, 3)
    BK_U8RRRROWS(1, 4, 512, 3)
    BK_U8RRRROWS(2, 1, 512, 3)
    BK_U8RRRROWS(4, 1, 512, 2)
    BK_U8RRRROWS(8, 1, 512, 2)
    BK_U8RRRROWS(2, 2, 512, 3)
    BK_U8RRRROWS(4, 2, 512, 2)
    BK_U8RRRROWS(8, 2, 512, 2)
    BK_U8RRRROWS(2, 4, 512, 3)
    BK_U8RRRROWS(4, 4, 512, 2)
    BK_U8RRRROWS(8, 4, 256, 2)
#undef BK_U8RRRROWS
    return false;
}

template <int ACT, typename BiasT>
int32_t launch_u8_rrr(const S8Args &p, hipStream_t stream, void *workspace = nullptr, size_t workspace_bytes = 0) {
    if (launch_u8_rrr_rows<ACT, BiasT>(p, stream)) return launch_status();
    const bool dma = u8_rrr_dma_eligible(p);
    if (u8_rrr_prepass_eligible(p) && workspace && workspace_bytes >= u8_rrr_workspace_bytes(p.M, p.N, p.K) &&
        (reinterpret_cast<uintptr_t>(workspace) & 255u) == 0) {
        int *rowsum = static_cast<int *>(workspace), *colsum = rowsum + p.M;
        int8_t *af = static_cast<int8_t *>(workspace) + u8_ws_sums_bytes(p.M, p.N);
        int8_t *bf = af + (((size_t)p.M * p.K + 255) & ~(size_t)255);
        const int agrid = max((p.M + 3) / 4, (p.N + 255) / 256);
        hipLaunchKernelGGL(u8_prep_a_kernel, dim3(agrid), dim3(256), 0, stream, (const uint8_t *)p.a, p.lda, p.M,
                           p.K, af, rowsum, colsum, p.N);
        hipLaunchKernelGGL(u8_prep_b_kernel, dim3((p.N + 255) / 256, (p.K + kU8ColSlice - 1) / kU8ColSlice),
                           dim3(256), 0, stream, (const uint8_t *)p.b, p.ldb, p.K, p.N, bf, colsum);
        S8Args q = p;
        q.a = af;
        q.lda = p.K;
        q.b = bf;
        q.ldb = p.N;
        const int tiles = (p.M / mfma2::BM) * (p.N / mfma2::BN);
        const bool vec = p.ldd % 4 == 0 && (reinterpret_cast<uintptr_t>(p.d) % 4) == 0;
        if (vec)
            hipLaunchKernelGGL((gemm_u8_rrr_ws_kernel<true, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0,
                               stream, q, (const int *)rowsum, (const int *)colsum);
        else
            hipLaunchKernelGGL((gemm_u8_rrr_ws_kernel<false, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0,
                               stream, q, (const int *)rowsum, (const int *)colsum);
        return launch_status();
    }
    if (dma) {
        const int tiles = (p.M / mfma2::BM) * (p.N / mfma2::BN);
        const bool vec = p.ldd % 4 == 0 && (reinterpret_cast<uintptr_t>(p.d) % 4) == 0;
        if (vec)
            hipLaunchKernelGGL((gemm_u8_rrr_dma_kernel<true, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0,
                               stream, p);
        else
            hipLaunchKernelGGL((gemm_u8_rrr_dma_kernel<false, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0,
                               stream, p);
        return launch_status();
    }
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    const bool aligned = p.K % BK == 0 && p.N % BN == 0 && p.lda % 16 == 0 && p.ldb % 4 == 0 &&
                         aligned16(p.a) && (reinterpret_cast<uintptr_t>(p.b) & 3u) == 0;
    if (aligned)
        hipLaunchKernelGGL((gemm_u8_rrr_kernel<true, ACT, BiasT>), dim3(tiles), dim3(NT), 0, stream, p);
    else
        hipLaunchKernelGGL((gemm_u8_rrr_kernel<false, ACT, BiasT>), dim3(tiles), dim3(NT), 0, stream, p);
    return launch_status();
}

// ---- u8 x u8 RCR (B [N, K]) ---------------------------------------------------
// Same correction as the RRR kernels; both operands are K-contiguous rows, so
// the column sums are B row sums, gathered exactly like the A row sums.
template <bool VecOut, int ACT, typename BiasT>
__global__ __launch_bounds__(DmaCfg::NT, 1) void gemm_u8_rcr_dma_kernel(S8Args p) {
    namespace M2 = mfma2;
    typedef M2::PolicyU8<DmaCfg> P;
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
    typename P::Sums sums;
    sums.ra = sums.rb = 0;
    M2::mainloop<P>(stage0, stage1, d, p.K, acc, sums);
    // Row sums of A and of B into LDS (free after the loop's last barrier),
    // above the staged-store scratch of waves 4..7 (stage1's first 32 KiB).
    int *sc = reinterpret_cast<int *>(stage1 + 40 * 1024);   // rs[256] | cs[256]
    park_row_sums(sums.ra, sc);
    park_row_sums(sums.rb, sc + 256);
    __syncthreads();
    const U8Epilogue<VecOut, ACT, BiasT> epi{p, sc, sc + 256, 16384u * (uint32_t)p.K};
    store_u8_tile<VecOut, P>(acc, stage0, stage1, p, m_base, n_base, epi);
}

// General u8 RCR path: register-staged mainloop, clamped rows, byte-exact K
// tail (zero-padded k: 0 in the raw sums, (-128)^2 in acc_s, K_pad corrects).
template <bool Aligned, int ACT, typename BiasT>
__global__ __launch_bounds__(NT, 1) void gemm_u8_rcr_kernel(S8Args p) {
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
    v4i acc[TM][TN];
    U8Sums sums;
    mainloop<Elem::U8, !Aligned>(lds, as, bs, p.K, acc, &sums);
    int *sc = reinterpret_cast<int *>(lds);
    park_row_sums(sums.ra, sc);
    park_row_sums(sums.cb, sc + 256);
    __syncthreads();
    const uint32_t kpad = (uint32_t)((p.K + BK - 1) / BK) * (uint32_t)BK;
    const U8Epilogue<false, ACT, BiasT> epi{p, sc, sc + 256, 16384u * kpad};
    for_each_fragment(acc, [&](int ml, int nl, const v4i &v) { epi(ml, nl, v, m_base, n_base); });
}

// u8 RCR last rows (decode-sized M; M % 256 in [1, 128] when a row of tiles
// would start another round) through the staged last-rows kernel; false
// when the shape does not fit it.  N = K = 4096: M = 1 / 16 / 128 on the
// register-staged general kernel took 68.9 / 68.1 / – us.
template <int ACT, typename BiasT>
bool launch_u8_rcr_rows(const S8Args &p, hipStream_t stream) {
    int rem = mfma2::last_rows_pass(p.M, p.N, 128), blocks = 1;
    bool whole = false;
    if (rem == 0 && p.M <= 512 && p.N % 16 == 0) {
        // a small grid of 256-row tiles: all rows as 128-row blocks of the
        // last-rows kernel.  N = K = 4096: M = 200 / 256 / 384 / 512 in
        // 28.1 / 26.8 / 38.6 / 49.1 us against 65-69 on the tiles
        rem = 128;
        blocks = (p.M + 127) / 128;
        whole = true;
    }
    if (rem == 0 || p.K % 512 != 0 || p.lda % 16 != 0 || p.ldb % 16 != 0 || !aligned16(p.a) || !aligned16(p.b) ||
        !dma_extent_ok(p.M, p.lda) || !dma_extent_ok(p.N, p.ldb))
        return false;
    S8Args pm = p;
    pm.M = whole ? 0 : p.M - rem;
    if (pm.M > 0 && p.N % mfma2::BN != 0) return false;
    const bool vec = p.ldd % 4 == 0 && (reinterpret_cast<uintptr_t>(p.d) % 4) == 0;
    if (pm.M > 0) {
        const int tiles = (pm.M / mfma2::BM) * (p.N / mfma2::BN);
        if (vec)
            hipLaunchKernelGGL((gemm_u8_rcr_dma_kernel<true, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0, stream, pm);
        else
            hipLaunchKernelGGL((gemm_u8_rcr_dma_kernel<false, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0, stream, pm);
    }
    if (rem == 1 && !whole && p.K % 1024 == 0) {
        // one row: the dot4 row kernel (N = K = 4096: 7.6 us on the staged kernel)
        if (p.K % 2048 == 0) {
            if (vec) hipLaunchKernelGGL((gemm_s8_rcr_row1_kernel<0, true, ACT, BiasT, 2, true>), dim3(p.N / 4), dim3(256), 0, stream, p, pm.M);
            else hipLaunchKernelGGL((gemm_s8_rcr_row1_kernel<0, false, ACT, BiasT, 2, true>), dim3(p.N / 4), dim3(256), 0, stream, p, pm.M);
        } else {
            if (vec) hipLaunchKernelGGL((gemm_s8_rcr_row1_kernel<0, true, ACT, BiasT, 1, true>), dim3(p.N / 4), dim3(256), 0, stream, p, pm.M);
            else hipLaunchKernelGGL((gemm_s8_rcr_row1_kernel<0, false, ACT, BiasT, 1, true>), dim3(p.N / 4), dim3(256), 0, stream, p, pm.M);
        }
        return true;
    }
    int rf, nb;
    rows_blocks_plan(p.M, p.N, rem, whole, rf, blocks, nb);
#define BK_U8ROWS(RF, NB, SB, DEPTH)                                                                           \
    if (rf == (RF) && nb == (NB)) {                                                                              \
        const size_t lds = std::max((size_t)(DEPTH) * (16 * (RF) + 16 * (NB)) * (SB), (size_t)(RF) * (NB) * ((SB) / 64) * 1024); \
        if (vec)                                                                                                \
            hipLaunchKernelGGL((gemm_s8_rcr_rows_staged_kernel<0, true, ACT, BiasT, RF, NB, SB, DEPTH, true>),    \
                               dim3(p.N / (16 * (NB)), blocks), dim3(1024), lds, stream, p, pm.M);                      \
        else                                                                                                    \
            hipLaunchKernelGGL((gemm_s8_rcr_rows_staged_kernel<0, false, ACT, BiasT, RF, NB, SB, DEPTH, true>),   \
                               dim3(p.N / (16 * (NB)), blocks), dim3(1024), lds, stream, p, pm.M);                      \
        return true;                                                                                            \
    }
    BK_U8ROWS(1, 1, 512, 3)
    BK_U8ROWS(1, 2, 512, 3)
    BK_U8ROWS(1, 4, 512, 3)
    BK_U8ROWS(2, 1, 512, 3)
    BK_U8ROWS(4, 1, 512, 2)
    BK_U8ROWS(8, 1, 512, 2)
    BK_U8ROWS(2, 2, 512, 3)
    BK_U8ROWS(4, 2, 512, 2)
    BK_U8ROWS(8, 2, 512, 2)
    BK_U8ROWS(2, 4, 512, 3)
    BK_U8ROWS(4, 4, 512, 2)
    BK_U8ROWS(8, 4, 256, 2)
#undef BK_U8ROWS
    return false;
}

template <int ACT, typename BiasT>
int32_t launch_u8_rcr(const S8Args &p, hipStream_t stream) {
    if (launch_u8_rcr_rows<ACT, BiasT>(p, stream)) return launch_status();
    const bool dma = p.K % mfma2::BK == 0 && p.M % mfma2::BM == 0 && p.N % mfma2::BN == 0 &&
                     p.lda % 16 == 0 && p.ldb % 16 == 0 && aligned16(p.a) && aligned16(p.b) &&
                     (int64_t)p.M * p.lda < (1ll << 31) && (int64_t)p.N * p.ldb < (1ll << 31);
    if (dma) {
        const int tiles = (p.M / mfma2::BM) * (p.N / mfma2::BN);
        const bool vec = p.ldd % 4 == 0 && (reinterpret_cast<uintptr_t>(p.d) % 4) == 0;
        if (vec)
            hipLaunchKernelGGL((gemm_u8_rcr_dma_kernel<true, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0,
                               stream, p);
        else
            hipLaunchKernelGGL((gemm_u8_rcr_dma_kernel<false, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0,
                               stream, p);
        return launch_status();
    }
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    const bool aligned = p.K % BK == 0 && p.lda % 16 == 0 && p.ldb % 16 == 0 && aligned16(p.a) &&
                         aligned16(p.b);
    if (aligned)
        hipLaunchKernelGGL((gemm_u8_rcr_kernel<true, ACT, BiasT>), dim3(tiles), dim3(NT), 0, stream, p);
    else
        hipLaunchKernelGGL((gemm_u8_rcr_kernel<false, ACT, BiasT>), dim3(tiles), dim3(NT), 0, stream, p);
    return launch_status();
}

template <int EPI, bool VecOut, int ACT, typename BiasT>
void launch_kernel(const S8Args &p, bool fast_k, hipStream_t stream, void *workspace, size_t workspace_bytes) {
    if (fast_k) {
        TailSplit ts = tail_split_plan(p.M, p.N, p.K);
        const size_t need = tail_split_workspace(p.M, p.N, p.K);
        const bool split_ws = ts.split > 1 && workspace != nullptr && workspace_bytes >= need &&
                              (reinterpret_cast<uintptr_t>(workspace) & 15u) == 0;
        const int rem = split_ws ? 0 : rows_path_rows(p.M, p.N);
        // Small problems (129-512 rows) whose 128-row blocks of the staged
        // last-rows kernel fit one round of workgroups run that way instead of
        // tiles.  K = 4096, M = 129 / 256 / 512: N = 4096 12.8 / 13.4 / 17.9 us
        // against 24.2 / 24.4 / 25.1 on 128x128 tiles; at N = 14336 the blocks
        // need 2-4 rounds and lose from 384 rows (48.9 against 37.0).
        // 64-row blocks first, when they still fit one round of workgroups
        // (K = 4096, M = 129 / 256: N = 4096 12.5 / 13.0 -> 11.0 / 11.4 us;
        // N = 2048 9.8 / 10.3 -> 7.6 / 7.8 us, M = 512 12.1 -> 10.9 us; N =
        // 8192 level).  Letting the 128-row blocks run two rounds was mixed
        // (N = 14336, M = 129: 34.6 -> 32.7 us; N = 6144, M = 384: 25.2 ->
        // 31.7 us), so they keep one.
        if (rem == 0 && !split_ws && p.M > 128 && p.M <= 512 && p.N % 16 == 0 && p.K % 512 == 0) {
            const int b4 = (p.M + 63) / 64;
            const int n4 = mfma2::last_rows_col_frags(p.N, b4);
            if (b4 * (p.N / (16 * n4)) <= 256) {
#define BK_S8BLK4(NB)                                                                                        \
                if (n4 == (NB)) {                                                                            \
                    hipLaunchKernelGGL((gemm_s8_rcr_rows_staged_kernel<EPI, VecOut, ACT, BiasT, 4, NB, 512, 2>), \
                                       dim3(p.N / (16 * (NB)), b4), dim3(1024),                              \
                                       std::max((size_t)2 * (64 + 16 * (NB)) * 512, (size_t)4 * (NB) * 8 * 1024), \
                                       stream, p, 0);                                                        \
                    return;                                                                                  \
                }
                BK_S8BLK4(1) BK_S8BLK4(2) BK_S8BLK4(4)
#undef BK_S8BLK4
            }
        }
        const int blocks = (p.M + 127) / 128;
        const int nbb = mfma2::last_rows_col_frags(p.N, blocks);
        if (rem == 0 && !split_ws && p.M > 128 && p.M <= 512 && p.N % 16 == 0 && p.K % 512 == 0 &&
            blocks * (p.N / (16 * nbb)) <= 256) {
            const int nb = nbb;
#define BK_S8BLOCKS(NB, SB)                                                                                  \
            if (nb == (NB)) {                                                                                \
                const size_t lds = std::max((size_t)2 * (128 + 16 * (NB)) * (SB), (size_t)8 * (NB) * ((SB) / 64) * 1024); \
                hipLaunchKernelGGL((gemm_s8_rcr_rows_staged_kernel<EPI, VecOut, ACT, BiasT, 8, NB, SB, 2>),    \
                                   dim3(p.N / (16 * (NB)), blocks), dim3(1024), lds, stream, p, 0);          \
                return;                                                                                      \
            }
            BK_S8BLOCKS(1, 512)
            BK_S8BLOCKS(2, 512)
            BK_S8BLOCKS(4, 256)
#undef BK_S8BLOCKS
        }
        if (rem != 0) {
            // whole 256-row tiles, then the last rows (gemm_s8_rcr_rows_kernel)
            S8Args pm = p;
            pm.M = p.M - rem;
            const int tiles = (pm.M / mfma2::BM) * ((p.N + mfma2::BN - 1) / mfma2::BN);
            if (tiles > 0)
                hipLaunchKernelGGL((gemm_s8_rcr_dma_kernel<EPI, VecOut, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT),
                                   0, stream, pm, TailSplit{0, 0, 1}, (int32_t *)nullptr);
            // fast_k already holds A and B 16-byte aligned, lda and ldb multiples
            // of 16 and both extents (rows rounded up to 256) below 2^31
            // With 32- or 64-column workgroups the staged kernel also beats the
            // B-only DMA kernel from 9 rows (N = 14336, K = 4096: M = 8 / 16
            // 14.3 / 17.5 us on the DMA kernel, 14.5 us staged at 17 rows).
            const int nb = mfma2::last_rows_col_frags(p.N);
            if (nb == 1 && rem > 32 && p.K % 512 == 0) {
                // 33-128 rows where 16-column workgroups would each read all
                // of them: 2-4 row blocks (last_rows_blocks).  K = 4096,
                // rotated weights, graph replay: N = 4096, M = 48 / 100 / 128
                // 8.5 / 11.6 / 11.9 -> 7.8 / 9.1 / 9.5 us; N = 2048, M = 48 /
                // 128 6.8 / 9.9 -> 5.8 / 6.5 us
                int rf, blk, nbb;
                mfma2::last_rows_blocks(rem, p.N, rf, blk, nbb);
#define BK_S8RBLK(RF, NB)                                                                                     \
                if (rf == (RF) && nbb == (NB)) {                                                               \
                    hipLaunchKernelGGL((gemm_s8_rcr_rows_staged_kernel<EPI, VecOut, ACT, BiasT, RF, NB, 512, 2>), \
                                       dim3(p.N / (16 * (NB)), blk), dim3(1024),                               \
                                       std::max((size_t)2 * (16 * (RF) + 16 * (NB)) * 512, (size_t)(RF) * (NB) * 8 * 1024), \
                                       stream, p, pm.M);                                                       \
                    return;                                                                                    \
                }
                BK_S8RBLK(2, 1) BK_S8RBLK(4, 1) BK_S8RBLK(2, 2) BK_S8RBLK(4, 2) BK_S8RBLK(2, 4) BK_S8RBLK(4, 4)
#undef BK_S8RBLK
            }
            if (nb == 1 && rem > 10 && rem <= 16 && p.K % 512 == 0) {
                // 11-16 rows below N = 6144: one fragment, 8 waves multiplying
                // (K = 4096, M = 12 / 16: N = 4096 6.55 / 6.93 -> 6.37 /
                // 6.42 us, N = 2048 4.95 / 5.27 -> 4.87 / 4.90 us against the
                // B-through-LDS kernel, which stays ahead up to 8 rows)
                hipLaunchKernelGGL((gemm_s8_rcr_rows_staged_kernel<EPI, VecOut, ACT, BiasT, 1, 1, 512, 3>),
                                   dim3(p.N / 16), dim3(1024), (size_t)3 * 32 * 512, stream, p, pm.M);
                return;
            }
            // staged from 6 rows at 64 columns (one fragment: N = 14336 / 12288,
            // M = 8 14.2 / 11.6 -> 13.2 / 10.8 us against the B-through-LDS
            // kernel, level at 2-5 rows), from 9 at 32 columns, from 17 at 16
            if (rem > (nb > 1 ? (nb == 4 ? 5 : 8) : kRowsDmaMaxRows) && p.K % kRowsStagedSB == 0) {
#define BK_S8ROWS(RF, NB, SB, DEPTH)                                                                        \
    if (rem <= 16 * (RF) && nb == (NB) && p.K % (SB) == 0) {                                                 \
        hipLaunchKernelGGL((gemm_s8_rcr_rows_staged_kernel<EPI, VecOut, ACT, BiasT, RF, NB, SB, DEPTH>),     \
                           dim3(p.N / (16 * (NB))), dim3(1024),                                             \
                           std::max((size_t)(DEPTH) * (16 * (RF) + 16 * (NB)) * (SB), (size_t)(RF) * (NB) * ((SB) / 64) * 1024), \
                           stream, p, pm.M);                                                                \
        return;                                                                                             \
    }
                BK_S8ROWS(2, 1, 512, 3)
                BK_S8ROWS(4, 1, 512, 2)
                BK_S8ROWS(8, 1, 512, 2)
                // up to 16 rows from N = 6144: one fragment, 8 waves
                // multiplying (N = 14336 / 8192, M = 12-16: 13.85 / 8.6-8.7
                // -> 13.3 / 8.5 us against two fragments)
                BK_S8ROWS(1, 2, 512, 2)
                BK_S8ROWS(1, 4, 512, 2)
                BK_S8ROWS(2, 2, 512, 3)
                BK_S8ROWS(4, 2, 512, 2)
                BK_S8ROWS(8, 2, 512, 2)
                BK_S8ROWS(2, 4, 512, 3)
                BK_S8ROWS(4, 4, 512, 2)
                BK_S8ROWS(8, 4, 256, 2)
#undef BK_S8ROWS
            }
            if (rem == 1 && p.K % 1024 == 0) {
                if (p.K % 2048 == 0)
                    hipLaunchKernelGGL((gemm_s8_rcr_row1_kernel<EPI, VecOut, ACT, BiasT, 2>), dim3(p.N / 4), dim3(256),
                                       0, stream, p, pm.M);
                else
                    hipLaunchKernelGGL((gemm_s8_rcr_row1_kernel<EPI, VecOut, ACT, BiasT, 1>), dim3(p.N / 4), dim3(256),
                                       0, stream, p, pm.M);
                return;
            }
            if (rem <= kRowsDmaMaxRows && p.K % 1024 == 0 && p.K <= kRowsDmaMaxK) {
                // B rows; the 16 waves' partial sums reuse the same LDS
                const size_t lds = std::max((size_t)16 * p.K, (size_t)kRowsDmaWaves * 1024);
                hipLaunchKernelGGL((gemm_s8_rcr_rows_dma_kernel<EPI, VecOut, ACT, BiasT, 1>), dim3(p.N / 16),
                                   dim3(1024), lds, stream, p, pm.M);
                return;
            }
            const dim3 grid(p.N / 16), block(512);
            if (rem <= 16)
                hipLaunchKernelGGL((gemm_s8_rcr_rows_kernel<EPI, VecOut, ACT, BiasT, 1>), grid, block, 0, stream, p, pm.M);
            else if (rem <= 32)
                hipLaunchKernelGGL((gemm_s8_rcr_rows_kernel<EPI, VecOut, ACT, BiasT, 2>), grid, block, 0, stream, p, pm.M);
            else if (rem <= 64)
                hipLaunchKernelGGL((gemm_s8_rcr_rows_kernel<EPI, VecOut, ACT, BiasT, 4>), grid, block, 0, stream, p, pm.M);
            else
                hipLaunchKernelGGL((gemm_s8_rcr_rows_kernel<EPI, VecOut, ACT, BiasT, 8>), grid, block, 0, stream, p, pm.M);
            return;
        }
        const int tiles = ((p.M + mfma2::BM - 1) / mfma2::BM) * ((p.N + mfma2::BN - 1) / mfma2::BN);
        if (split_ws) {
            int32_t *slots = static_cast<int32_t *>(workspace);
            hipLaunchKernelGGL((gemm_s8_rcr_dma_kernel<EPI, VecOut, ACT, BiasT>),
                               dim3(ts.full_tiles + ts.tail_tiles * ts.split), dim3(DmaCfg::NT), 0, stream, p, ts,
                               slots);
            hipLaunchKernelGGL((gemm_s8_tail_reduce_kernel<EPI, VecOut, ACT, BiasT>), dim3(ts.tail_tiles, 64),
                               dim3(256), 0, stream, p, ts, (const int32_t *)slots);
            return;
        }
        if (tiles <= kSmallTilesMax) {
            typedef mfma2::Cfg<2, 2, 128> SmallCfg;
            const int tiles128 = ((p.M + 127) / 128) * ((p.N + 127) / 128);
            hipLaunchKernelGGL((gemm_s8_rcr_dma_kernel<EPI, VecOut, ACT, BiasT, SmallCfg>), dim3(tiles128),
                               dim3(SmallCfg::NT), 0, stream, p, TailSplit{0, 0, 1}, (int32_t *)nullptr);
            return;
        }
        hipLaunchKernelGGL((gemm_s8_rcr_dma_kernel<EPI, VecOut, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0, stream, p,
                           TailSplit{0, 0, 1}, (int32_t *)nullptr);
    } else {
        const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
        hipLaunchKernelGGL((gemm_s8_rcr_kernel<EPI, VecOut, ACT, BiasT>), dim3(tiles), dim3(NT), 0, stream, p);
    }
}

// workspace (optional): tail_split_workspace(M, N, K) bytes, 16-byte aligned,
// contents on entry do not matter; given it, a partial last round of tiles
// runs split along K (tail_split_plan).
template <int EPI, int ACT = ACT_NONE, typename BiasT = float>
int32_t launch(const S8Args &p, hipStream_t stream, void *workspace = nullptr, size_t workspace_bytes = 0) {
    const int out_elem = (EPI == EPI_I32 || EPI == EPI_W8A8_F32) ? 4 : EPI == EPI_W8A8_F64 ? 8 : (EPI == EPI_S8 ? 1 : 2);
    // The DMA path needs whole K stages and 16-byte rows; edge tiles read
    // zeros past the operands, so the byte offsets of the padded extents
    // must stay below 2^31.
    const bool fast_k = p.K > 0 && p.K % BK == 0 && p.lda % 16 == 0 && p.ldb % 16 == 0 &&
                        aligned16(p.a) && aligned16(p.b) && dma_extent_ok(p.M, p.lda) &&
                        dma_extent_ok(p.N, p.ldb);
    // 4-wide vector stores need every 4-column group of D (and sw) aligned;
    // the LDS-staged W8A8 bf16 store writes 16-byte units (8 columns).
    bool vec = ((p.ldd * out_elem) % (4 * out_elem)) == 0 &&
               (reinterpret_cast<uintptr_t>(p.d) % (4 * out_elem)) == 0 &&
               (p.sw == nullptr || aligned16(p.sw)) && (p.N % 4 == 0);
    if (EPI == EPI_W8A8_BF16) vec = vec && p.ldd % 8 == 0 && aligned16(p.d);
    if (vec) launch_kernel<EPI, true, ACT, BiasT>(p, fast_k, stream, workspace, workspace_bytes);
    else launch_kernel<EPI, false, ACT, BiasT>(p, fast_k, stream, workspace, workspace_bytes);
    return launch_status();
}

// Launches the RRR DMA kernel when the problem fits it (whole 256x256 tiles,
// K % 128 == 0, 16-byte A / B rows and bases, buffer offsets below 2^31);
// returns kOk if launched, kUnsupported to let the caller take the general
// kernel.
template <int ACT, typename BiasT>
int32_t launch_rrr_dma(const S8Args &p, hipStream_t stream) {
    const bool fits = p.K % mfma2::BK == 0 && p.lda % 16 == 0 && p.ldb % 16 == 0 && aligned16(p.a) &&
                      aligned16(p.b) && dma_extent_ok(p.M, p.lda) && (int64_t)p.K * p.ldb + mfma2::BN < (1ll << 31);
    if (!fits) return kUnsupported;
    const int tiles = ((p.M + mfma2::BM - 1) / mfma2::BM) * ((p.N + mfma2::BN - 1) / mfma2::BN);
    const bool vec = p.N % 4 == 0 && p.ldd % 4 == 0 && (reinterpret_cast<uintptr_t>(p.d) % 4) == 0;
    if (vec)
        hipLaunchKernelGGL((gemm_s8_rrr_dma_kernel<true, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0, stream, p);
    else
        hipLaunchKernelGGL((gemm_s8_rrr_dma_kernel<false, ACT, BiasT>), dim3(tiles), dim3(DmaCfg::NT), 0, stream, p);
    return kOk;
}

// s8 RRR last rows (decode-sized M; M % 256 in [1, 128] when a row of tiles
// would start another round): the staged last-rows kernel reading row-major
// B; false when the shape does not fit it (K % 512 == 0, 16-byte rows and
// bases, N % (16 NB) == 0, K * ldb below 2^31).
template <int ACT, typename BiasT>
bool launch_rrr_rows(const S8Args &p, hipStream_t stream) {
    int rem = mfma2::last_rows_pass(p.M, p.N, 128), blocks = 1;
    bool whole = false;
    if (rem == 0 && p.M <= 512 && p.N % 16 == 0) {
        // a small grid of 256-row tiles: all rows as 128-row blocks.  N = K =
        // 4096: M = 200 / 256 / 512 in 23.0 / 22.9 / 23.3 us against 44 on the
        // tiles; from 768 rows the blocks need a second round (44.6 on tiles)
        rem = 128;
        blocks = (p.M + 127) / 128;
        whole = true;
    }
    if (rem == 0 || p.K % 512 != 0 || p.lda % 16 != 0 || p.ldb % 16 != 0 || !aligned16(p.a) || !aligned16(p.b) ||
        !dma_extent_ok(p.M, p.lda) || (int64_t)p.K * p.ldb + mfma2::BN >= (1ll << 31))
        return false;
    // column groups by the last-rows rule (16 / 32 / 64 columns, at least 192
    // workgroups), numbered XCD-major in the kernel so the groups sharing a
    // B line share an L2: N = 4096 / 14336, K = 4096, M = 1: 9.6 / 15.3 us
    // (16 / 64 columns; 64 columns at N = 4096 13.1, 16 at N = 14336 23.1;
    // before the XCD-major numbering 64 columns 13.4 / 21.6; the 256x256 RRR
    // tiles 40.5 / 37.7)
    int rf, nb;
    rows_blocks_plan(p.M, p.N, rem, whole, rf, blocks, nb);
    S8Args pm = p;
    pm.M = whole ? 0 : p.M - rem;
    if (pm.M > 0 && launch_rrr_dma<ACT, BiasT>(pm, stream) != kOk) return false;
    const bool vec = p.N % 4 == 0 && p.ldd % 4 == 0 && (reinterpret_cast<uintptr_t>(p.d) % 4) == 0;
#define BK_RRRROWS(RF, NB, SB, DEPTH)                                                                          \
    if (rf == (RF) && nb == (NB)) {                                                                              \
        const size_t lds = std::max((size_t)(DEPTH) * (16 * (RF) + 16 * (NB)) * (SB), (size_t)(RF) * (NB) * ((SB) / 64) * 1024); \
        if (vec)                                                                                                \
            hipLaunchKernelGGL((gemm_s8_rcr_rows_staged_kernel<EPI_S8, true, ACT, BiasT, RF, NB, SB, DEPTH, false, true>), \
                               dim3(p.N / (16 * (NB)), blocks), dim3(1024), lds, stream, p, pm.M);                      \
        else                                                                                                    \
            hipLaunchKernelGGL((gemm_s8_rcr_rows_staged_kernel<EPI_S8, false, ACT, BiasT, RF, NB, SB, DEPTH, false, true>), \
                               dim3(p.N / (16 * (NB)), blocks), dim3(1024), lds, stream, p, pm.M);                      \
        return true;                                                                                            \
    }
    BK_RRRROWS(1, 1, 512, 3)
    BK_RRRROWS(1, 2, 512, 3)
    BK_RRRROWS(1, 4, 512, 3)
    BK_RRRROWS(2, 1, 512, 3)
    BK_RRRROWS(4, 1, 512, 2)
    BK_RRRROWS(8, 1, 512, 2)
    BK_RRRROWS(2, 2, 512, 3)
    BK_RRRROWS(4, 2, 512, 2)
    BK_RRRROWS(8, 2, 512, 2)
    BK_RRRROWS(2, 4, 512, 3)
    BK_RRRROWS(4, 4, 512, 2)
    BK_RRRROWS(8, 4, 256, 2)
#undef BK_RRRROWS
    return false;
}

int32_t check_rcr(int32_t m, int32_t n, int32_t k, int64_t lda, int64_t ldb, int64_t ldd) {
    if (m <= 0 || n <= 0 || k <= 0) return kInvalid;
    if (lda < k || ldb < k || ldd < n) return kInvalid;
    return kOk;
}

}  // namespace
}  // namespace bk

