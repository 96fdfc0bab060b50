// gemm_mfma.hpp -- the gfx950 MFMA mainloop shared by the int8 and FP8 RCR
// GEMMs and the grouped MoE GEMM.
//
// Problem: C[m,n] = sum_k A[m,k] * B[n,k] with A row-major [M,K] (lda) and B
// "column-major [K,N]" = row-major [N,K] (ldb).  Both operands are
// K-contiguous, which is exactly what the MFMA operand registers want.
//
// Block tile 256(M) x 256(N) x 128(K) bytes, 512 threads = 8 wave64s laid
// out 2 (M) x 4 (N); each wave owns a 128 x 64 output tile held as 8 x 4
// MFMA 16x16 accumulators (128 VGPRs).
//
// LDS: A and B tiles are [256 rows][128 bytes], double buffered (128 KiB).
// Rows are 128 B, so every row starts on the same bank; the 16-byte unit u
// of row r is stored at unit u ^ swz(r), swz(r) = (r >> 1) & 7, the XOR
// pattern measured bank-conflict free on gfx950 for these ds_read_b128 /
// ds_write_b128 patterns.
//
// This register-staged mainloop serves the general case (K tail, unaligned
// rows); aligned problems take the LDS-DMA mainloop of gemm_mfma2.hpp.
//
// MFMA operand roles are swapped (srcA = B rows, srcB = A rows) so the
// 16x16 result lane l holds C[m = l%16][n = 4*(l/16) + r], r = 0..3: four
// consecutive output columns per lane, i.e. one 8-byte bf16 (16-byte i32)
// store per 16x16 tile.
//
// Both operand fragments use the same lane -> (row, k-chunk) mapping, so
// every k of the block is paired with itself in A and B whatever the
// intra-instruction K order of the hardware is: integer results are exact.
#pragma once

#include "bk_common.hpp"

namespace bk {
namespace mfma {

constexpr int BM = 256;
constexpr int BN = 256;
constexpr int BK = 128;             // bytes of K per pipeline stage
constexpr int NT = 512;             // threads per block
constexpr int WAVES_M = 2;
constexpr int WAVES_N = 4;
constexpr int WM = BM / WAVES_M;    // 128
constexpr int WN = BN / WAVES_N;    // 64
constexpr int TM = WM / 16;         // 8 MFMA tiles along M per wave
constexpr int TN = WN / 16;         // 4 MFMA tiles along N per wave
constexpr int LDS_TILE = BM * BK;   // 32 KiB per operand per stage
constexpr int LOAD_ROWS = NT / 8;   // rows covered by one 16-byte load wave (64)
constexpr int LOADS = BM / LOAD_ROWS;  // 4 loads per operand per stage

__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

__device__ __forceinline__ int lds_off(int row, int unit) {
    return row * BK + ((unit ^ swz(row)) << 4);
}

enum class Elem { S8, U8, E4M3, E5M2, BF16, F16 };

template <Elem E> struct AccT { typedef v4f type; };   // FP8: f32 accumulators
template <> struct AccT<Elem::S8> { typedef v4i type; };
template <> struct AccT<Elem::U8> { typedef v4i type; };

// u8 operands through the signed int8 MFMA: fragments are flipped to
// s = u - 128 (xor 0x80 per byte) right before the MFMA, and once per stage
// each wave sums the raw bytes of its slice of the LDS tile: rows
// 32*wave .. +31 of A and of B (stored [n][k]), two lanes per row.  The
// epilogue restores sum(u_a*u_b) = acc_s + 128*(rowsum + colsum) - 16384*K_pad
// (zero-padded k are 0 in the raw sums and -128*-128 in acc_s).
struct U8Sums {
    uint32_t ra;   // raw-byte sum, A row 32*wave + lane/2, half lane%2 of each stage
    uint32_t cb;   // the same for B row (= output column) 32*wave + lane/2
};

// Per-thread view of the rows this thread stages into LDS.  Each of the 4
// loads of a stage covers row (i * 64 + tid / 8), 16-byte unit tid % 8.
// Rows past the end of the problem point at a valid row (the caller clamps
// them) and their results are never stored, so loads need no row guard.
struct RowSet {
    const int8_t *ptr[LOADS];   // start of the row (k = 0)
};

// Load one 16-byte chunk at byte k of a row of length K bytes.  Checked
// handles a K tail and rows that are not 16-byte aligned.
template <bool Checked>
__device__ __forceinline__ v4i load_chunk(const int8_t *row, int k, int K) {
    if constexpr (!Checked) {
        return *reinterpret_cast<const v4i *>(row + k);
    } else {
        v4i v = {0, 0, 0, 0};
        if (k >= K) return v;
        if (k + 16 <= K && ((reinterpret_cast<uintptr_t>(row + k) & 15u) == 0)) {
            return *reinterpret_cast<const v4i *>(row + k);
        }
        uint32_t w[4] = {0, 0, 0, 0};
        for (int b = 0; b < 16; ++b) {
            if (k + b < K) w[b >> 2] |= (uint32_t)(uint8_t)row[k + b] << ((b & 3) * 8);
        }
        v[0] = (int)w[0]; v[1] = (int)w[1]; v[2] = (int)w[2]; v[3] = (int)w[3];
        return v;
    }
}

template <bool Checked>
__device__ __forceinline__ void load_stage(v4i (&ra)[LOADS], v4i (&rb)[LOADS],
                                           const RowSet &as, const RowSet &bs,
                                           int kbyte, int K, int unit) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) ra[i] = load_chunk<Checked>(as.ptr[i], kbyte + unit * 16, K);
#pragma unroll
    for (int i = 0; i < LOADS; ++i) rb[i] = load_chunk<Checked>(bs.ptr[i], kbyte + unit * 16, K);
}

__device__ __forceinline__ void store_stage(int8_t *la, int8_t *lb, const v4i (&ra)[LOADS],
                                            const v4i (&rb)[LOADS], int tid) {
    const int unit = tid & 7;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int row = i * LOAD_ROWS + (tid >> 3);
        *reinterpret_cast<v4i *>(la + lds_off(row, unit)) = ra[i];
        *reinterpret_cast<v4i *>(lb + lds_off(row, unit)) = rb[i];
    }
}

// One 128-byte K stage of MFMA work for this wave.
template <Elem E>
__device__ __forceinline__ void compute_stage(const int8_t *la, const int8_t *lb,
                                              typename AccT<E>::type (&acc)[TM][TN],
                                              int wave_m, int wave_n, int lane,
                                              U8Sums *sums = nullptr) {
    const int r16 = lane & 15;
    const int grp = lane >> 4;
    if constexpr (E == Elem::S8 || E == Elem::U8 || E == Elem::BF16 || E == Elem::F16) {
        // v_mfma_i32_16x16x64_i8 / v_mfma_f32_16x16x32_{bf16,f16}: 16 bytes of
        // K per lane, 2 sub-steps per stage.
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int unit = s * 4 + grp;
            v4i bf[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int row = wave_n * WN + j * 16 + r16;
                bf[j] = *reinterpret_cast<const v4i *>(lb + lds_off(row, unit));
                if constexpr (E == Elem::U8) bf[j] = u8_flip(bf[j]);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int row = wave_m * WM + i * 16 + r16;
                v4i af = *reinterpret_cast<const v4i *>(la + lds_off(row, unit));
                if constexpr (E == Elem::U8) af = u8_flip(af);
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if constexpr (E == Elem::BF16 || E == Elem::F16)
                        acc[i][j] = mfma16x16x32_h<E == Elem::BF16>(bf[j], af, acc[i][j]);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[j], af, acc[i][j], 0, 0, 0);
                }
            }
        }
        if constexpr (E == Elem::U8) {
            // Raw-byte sums of this wave's slice of the stage (fragments dead here).
            const int row = 32 * (threadIdx.x >> 6) + (lane >> 1);
            const int u0 = (lane & 1) * 4;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                sums->ra = u8_sum16(*reinterpret_cast<const v4i *>(la + lds_off(row, u0 + u)), sums->ra);
                sums->cb = u8_sum16(*reinterpret_cast<const v4i *>(lb + lds_off(row, u0 + u)), sums->cb);
            }
        }
    } else {
        // v_mfma_f32_16x16x128_f8f6f4 (cbsz = blgp = 0: e4m3 x e4m3, 1: e5m2 x
        // e5m2): 32 bytes of K per lane, one instruction covers the stage.
        constexpr int F = E == Elem::E5M2 ? 1 : 0;
        const int u0 = grp * 2;
        v8i bf[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int row = wave_n * WN + j * 16 + r16;
            v4i lo = *reinterpret_cast<const v4i *>(lb + lds_off(row, u0));
            v4i hi = *reinterpret_cast<const v4i *>(lb + lds_off(row, u0 + 1));
            bf[j] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int row = wave_m * WM + i * 16 + r16;
            v4i lo = *reinterpret_cast<const v4i *>(la + lds_off(row, u0));
            v4i hi = *reinterpret_cast<const v4i *>(la + lds_off(row, u0 + 1));
            v8i af = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                    bf[j], af, acc[i][j], F, F, 0, 0, 0, 0);
        }
    }
}

// Full K loop for one 256x256 output tile.  `lds` must hold 2 * 2 * LDS_TILE
// bytes.  Ends with a barrier so the caller may reuse LDS.
// U8 needs `sums` (zeroed here): raw-byte sums of A rows and B rows (= output
// columns), gathered by compute_stage.
template <Elem E, bool Checked>
__device__ __forceinline__ void mainloop(int8_t *lds, const RowSet &as, const RowSet &bs, int K,
                                         typename AccT<E>::type (&acc)[TM][TN],
                                         U8Sums *sums = nullptr) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave / WAVES_N;
    const int wave_n = wave % WAVES_N;
    const int unit = tid & 7;

#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = typename AccT<E>::type{0, 0, 0, 0};

    if constexpr (E == Elem::U8) sums->ra = sums->cb = 0;
    const int KT = (K + BK - 1) / BK;
    v4i ra[LOADS], rb[LOADS];
    load_stage<Checked>(ra, rb, as, bs, 0, K, unit);
    store_stage(lds, lds + LDS_TILE, ra, rb, tid);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        int8_t *cur = lds + (kt & 1) * 2 * LDS_TILE;
        int8_t *nxt = lds + ((kt + 1) & 1) * 2 * LDS_TILE;
        const bool more = kt + 1 < KT;
        if (more) load_stage<Checked>(ra, rb, as, bs, (kt + 1) * BK, K, unit);
        compute_stage<E>(cur, cur + LDS_TILE, acc, wave_m, wave_n, lane, sums);
        if (more) store_stage(nxt, nxt + LDS_TILE, ra, rb, tid);
        __syncthreads();
    }
}

// Visit this thread's accumulator fragments: f(m, n0, acc) where m is the
// tile-local row and n0 the tile-local first of the 4 consecutive columns
// held in acc[0..3].
template <class AccV, class F>
__device__ __forceinline__ void for_each_fragment(const AccV (&acc)[TM][TN], F &&f) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wave_m = wave / WAVES_N, wave_n = wave % WAVES_N;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int m = wave_m * WM + i * 16 + (lane & 15);
#pragma unroll
        for (int j = 0; j < TN; ++j) f(m, wave_n * WN + j * 16 + (lane >> 4) * 4, acc[i][j]);
    }
}

// Packs 4 floats to 4 bf16 (RNE) and stores 8 bytes, or element-wise when
// the destination is not 8-byte aligned / runs past `count`.
__device__ __forceinline__ void store4_bf16(uint16_t *d, const float (&y)[4], bool vec, int count) {
    if (vec) {
        v2i w;
        w[0] = (int)f32x2_to_bf16x2(y[0], y[1]);
        w[1] = (int)f32x2_to_bf16x2(y[2], y[3]);
        *reinterpret_cast<v2i *>(d) = w;
    } else {
        for (int r = 0; r < 4; ++r) if (r < count) d[r] = f32_to_bf16_rne(y[r]);
    }
}

__device__ __forceinline__ void store4_f32(float *d, const float (&y)[4], bool vec, int count) {
    if (vec) {
        *reinterpret_cast<v4f *>(d) = (v4f){y[0], y[1], y[2], y[3]};
    } else {
        for (int r = 0; r < 4; ++r) if (r < count) d[r] = y[r];
    }
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- RRR: B is row-major [K, N] (n contiguous) ------------------------------
// Per stage the B tile (256 n x 128 k) is loaded transposed: thread t owns
// the 4 columns n = 4*(t % 64) .. +3 over the 16 rows k = 16*(t / 64) .. +15
// (16 dword loads, workgroup-coalesced along n), byte-transposes them in
// registers and writes 4 LDS rows of 16 k-bytes, so the LDS image is the same
// [n][k] tile the RCR path builds and compute_stage is shared.
template <bool Checked>
__device__ __forceinline__ void load_b_rrr(v4i (&rb)[LOADS], const int8_t *b, int64_t ldb, int N,
                                           int K, int n0, int kbyte, int tid) {
    const int n = n0 + 4 * (tid & 63);
    const int k0 = kbyte + 16 * (tid >> 6);
    uint32_t w[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int k = k0 + r;
        if constexpr (!Checked) {
            w[r] = *reinterpret_cast<const uint32_t *>(b + (int64_t)k * ldb + n);
        } else {
            uint32_t v = 0;
            if (k < K) {
                const int8_t *p = b + (int64_t)k * ldb;
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (n + c < N) v |= (uint32_t)(uint8_t)p[n + c] << (8 * c);
            }
            w[r] = v;
        }
    }
#pragma unroll
    for (int c = 0; c < LOADS; ++c) {
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            o[q] = ((w[4 * q] >> (8 * c)) & 0xffu) | (((w[4 * q + 1] >> (8 * c)) & 0xffu) << 8) |
                   (((w[4 * q + 2] >> (8 * c)) & 0xffu) << 16) | (((w[4 * q + 3] >> (8 * c)) & 0xffu) << 24);
        rb[c] = v4i{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
    }
}

__device__ __forceinline__ void store_b_rrr(int8_t *lb, const v4i (&rb)[LOADS], int tid) {
    const int unit = tid >> 6;                 // 16-byte k unit of the 128-byte row
#pragma unroll
    for (int c = 0; c < LOADS; ++c) {
        const int row = 4 * (tid & 63) + c;    // n within the tile
        *reinterpret_cast<v4i *>(lb + lds_off(row, unit)) = rb[c];
    }
}

// K loop for one 256x256 RRR tile (A as in mainloop, B through load_b_rrr).
// CheckedB: N tail / unaligned B rows / K tail on B.
template <Elem E, bool CheckedA, bool CheckedB>
__device__ __forceinline__ void mainloop_rrr(int8_t *lds, const RowSet &as, const int8_t *b,
                                             int64_t ldb, int N, int n0, int K,
                                             typename AccT<E>::type (&acc)[TM][TN],
                                             U8Sums *sums = nullptr) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave / WAVES_N;
    const int wave_n = wave % WAVES_N;
    const int unit = tid & 7;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = typename AccT<E>::type{0, 0, 0, 0};
    if constexpr (E == Elem::U8) sums->ra = sums->cb = 0;
    const int KT = (K + BK - 1) / BK;
    v4i ra[LOADS], rb[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) ra[i] = load_chunk<CheckedA>(as.ptr[i], unit * 16, K);
    load_b_rrr<CheckedB>(rb, b, ldb, N, K, n0, 0, tid);
    {
        const int row0 = tid >> 3;
#pragma unroll
        for (int i = 0; i < LOADS; ++i)
            *reinterpret_cast<v4i *>(lds + lds_off(i * LOAD_ROWS + row0, unit)) = ra[i];
        store_b_rrr(lds + LDS_TILE, rb, tid);
    }
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        int8_t *cur = lds + (kt & 1) * 2 * LDS_TILE;
        int8_t *nxt = lds + ((kt + 1) & 1) * 2 * LDS_TILE;
        const bool more = kt + 1 < KT;
        if (more) {
#pragma unroll
            for (int i = 0; i < LOADS; ++i) ra[i] = load_chunk<CheckedA>(as.ptr[i], (kt + 1) * BK + unit * 16, K);
            load_b_rrr<CheckedB>(rb, b, ldb, N, K, n0, (kt + 1) * BK, tid);
        }
        compute_stage<E>(cur, cur + LDS_TILE, acc, wave_m, wave_n, lane, sums);
        if (more) {
            const int row0 = tid >> 3;
#pragma unroll
            for (int i = 0; i < LOADS; ++i)
                *reinterpret_cast<v4i *>(nxt + lds_off(i * LOAD_ROWS + row0, unit)) = ra[i];
            store_b_rrr(nxt + LDS_TILE, rb, tid);
        }
        __syncthreads();
    }
}

// Tile index -> (tile_m, tile_n).  Consecutive workgroups are dispatched
// round-robin over the 8 XCDs, so the linear id is first regrouped so that
// each XCD gets a contiguous run of tiles, and runs are laid out in groups
// of GROUP_M tile-rows so an XCD's tiles share A row panels and B column
// panels in its own L2.
__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int &tm, int &tn) {
    constexpr int XCDS = 8;
    constexpr int GROUP_M = 4;
    const int total = tiles_m * tiles_n;
    int t = pid;
    if (total % XCDS == 0) t = (pid % XCDS) * (total / XCDS) + pid / XCDS;
    const int group_span = GROUP_M * tiles_n;
    const int g = t / group_span;
    const int first_m = g * GROUP_M;
    const int gsize = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
    const int in_g = t - g * group_span;
    tm = first_m + in_g % gsize;
    tn = in_g / gsize;
}

}  // namespace mfma
}  // namespace bk
