// gemm_mfma2.hpp -- the fast gfx950 MFMA mainloop (aligned problems) shared
// by the int8 / FP8 RCR GEMMs and the grouped MoE GEMM.
//
// C[m,n] = sum_k A[m,k] * B[n,k]; A row-major [M,K], B row-major [N,K] (the
// RCR "column-major [K,N]" operand).  Requirements checked by the launcher:
// K % 128 == 0, lda % 16 == 0, ldb % 16 == 0, 16-byte aligned bases.
//
// Block tile 256(M) x 256(N); Cfg<WAVES_M, WAVES_N> picks the wave
// grid (the int8 and FP8 kernels use 2 x 4 wave64s, each owning a 128 x 64
// output tile, two waves per SIMD).  K advances 128 bytes per stage, two
// stages in flight.
//
// Global -> LDS: direct DMA (global_load_lds_dwordx4), no staging registers.
// One DMA instruction writes 1 KiB of LDS linearly (lane L -> bytes 16L..16L+15)
// = 8 rows of 128 bytes; lane L fetches the logical 16-byte unit
// u = (L % 8) ^ swz(row) of row (L / 8), so the LDS image is the row-major
// tile with unit u of row r at physical unit u ^ swz(r).  swz(r) = (r >> 1) & 7
// is the XOR pattern measured bank-conflict free on gfx950 for every
// ds_read_b128 fragment pattern used below (16-row int8 and 32-row fp8 frags).
//
// Per stage and wave: the DMA of the next stage is issued into the other
// buffer, then 2 sub-steps of 64 bytes of K, each reading its fragments and
// issuing its MFMAs (the two waves of a SIMD interleave), then a wait for
// this wave's DMA and the stage's one barrier.  The two stage buffers are
// distinct __shared__ arrays and the loop is unrolled by two, so the DMA
// into one buffer is never mistaken for a write to the buffer being read
// (no spurious vmcnt waits before ds_reads).
//
// Both operand fragments use the same lane -> (row, k) mapping, so every k is
// paired with itself whatever the hardware's intra-instruction K order is:
// integer results are exact.
#pragma once

#include "bk_common.hpp"

namespace bk {
namespace mfma2 {

constexpr int BM = 256;
constexpr int BN = 256;
constexpr int BK = 128;
constexpr int OPER = BM * BK;        // 32 KiB per operand per stage

// Block configuration: WAVES_M x WAVES_N wave64s, each owning a
// (256 / WAVES_M) x (256 / WAVES_N) output tile.  Per sub-step a wave reads
// its fragments, then issues its MFMAs; the latency is hidden by the other
// wave of the SIMD.  (Measured slower and removed: double-buffered
// fragments, a mid-stage barrier, pinned read/MFMA interleaving, a
// ping-pong of the two waves of a SIMD, one wave per SIMD.)
// TB: square block tile edge (256 by default; the A and B stage regions are
// TB x BK bytes each, B at stage + OPER).
template <int WAVES_M_, int WAVES_N_, int TB_ = 256>
struct Cfg {
    static constexpr int WAVES_M = WAVES_M_;
    static constexpr int WAVES_N = WAVES_N_;
    static constexpr int TB = TB_;
    static constexpr int OPER = TB * BK;                    // bytes per operand per stage
    static constexpr int WAVES = WAVES_M * WAVES_N;
    static constexpr int NT = 64 * WAVES;
    static constexpr int WM = TB / WAVES_M;
    static constexpr int WN = TB / WAVES_N;
    static constexpr int ROWS_PER_WAVE = TB / WAVES;       // DMA rows per wave per operand
    static constexpr int DMA_PER_WAVE = ROWS_PER_WAVE / 8;  // 1 KiB DMA instructions
    static_assert(ROWS_PER_WAVE % 8 == 0, "whole 1 KiB DMA groups per wave");
};

typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int lds_off(int row, int unit) { return row * BK + ((unit ^ swz(row)) << 4); }

// ---------------------------------------------------------------------------
// MFMA policies
// ---------------------------------------------------------------------------
// int8: v_mfma_i32_16x16x64_i8.  Wave tile = 8 x 8 tiles of 16x16.
template <class C>
struct PolicyI8 {
    typedef C Cfg;
    static constexpr bool SUMS = false;   // u8 operand correction (PolicyU8RowB)
    static constexpr bool FLIP = false;   // u8 operands flipped to u - 128 (PolicyU8RowB)
    struct Sums {};
    template <class F> __device__ static void fixup(F &, Sums &) {}
    __device__ static void stage_hook(const int8_t *, Sums &) {}

    static constexpr int TI = C::WM / 16;    // 16x16 tiles per wave along M
    static constexpr int TJ = C::WN / 16;    // ... along N
    typedef v4i Acc;
    typedef v4i Frag;
    __device__ static Frag load(const int8_t *op, int row0, int t, int s, int lane) {
        const int row = row0 + t * 16 + (lane & 15);
        return *reinterpret_cast<const v4i *>(op + lds_off(row, s * 4 + (lane >> 4)));
    }
    __device__ static Frag load_b(const int8_t *op, int row0, int t, int s, int lane) {
        return load(op, row0, t, s, lane);
    }
    static constexpr int H = 1;
    __device__ static void mma(Acc &c, const Frag &b, const Frag &a, int) {
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(b, a, c, 0, 0, 0);
    }
    __device__ static Acc zero() { return Acc{0, 0, 0, 0}; }
    // Accumulator tile (i, j) -> groups of 4 consecutive columns.
    template <class F>
    __device__ static void visit(const Acc &c, int i, int j, int lane, F &&f) {
        f(i * 16 + (lane & 15), j * 16 + (lane >> 4) * 4, v4i{c[0], c[1], c[2], c[3]});
    }
};

// bf16 / f16: v_mfma_f32_16x16x32_{bf16,f16} takes the same 16 bytes of K
// per lane as the int8 16x16x64 form, so the fragment layout, swizzle and
// sub-step structure are PolicyI8's; only the instruction and the f32
// accumulators differ.
template <class C, bool IsBf16>
struct PolicyH16 : PolicyI8<C> {
    typedef v4f Acc;
    __device__ static void mma(Acc &c, const v4i &b, const v4i &a, int) { c = mfma16x16x32_h<IsBf16>(b, a, c); }
    __device__ static Acc zero() { return Acc{0.0f, 0.0f, 0.0f, 0.0f}; }
    template <class F>
    __device__ static void visit(const Acc &c, int i, int j, int lane, F &&f) {
        f(i * 16 + (lane & 15), j * 16 + (lane >> 4) * 4, c);
    }
};

// int8: v_mfma_i32_32x32x32_i8 (sustains ~25% more int8 ops/clk than the
// 16x16x64 form on gfx950 with random operands).  Wave tile = TI x TJ tiles
// of 32x32; a 64-byte sub-step of K is two instructions (h = 0, 1), lane l
// supplying row l % 32 and the 16-byte unit s*4 + 2h + l/32.
template <class C>
struct PolicyI8x32 {
    typedef C Cfg;
    static constexpr bool SUMS = false;   // u8 operand correction (PolicyU8RowB)
    static constexpr bool FLIP = false;   // u8 operands flipped to u - 128 (PolicyU8RowB)
    struct Sums {};
    template <class F> __device__ static void fixup(F &, Sums &) {}
    __device__ static void stage_hook(const int8_t *, Sums &) {}

    static constexpr int TI = C::WM / 32;
    static constexpr int TJ = C::WN / 32;
    typedef v16i Acc;
    struct Frag { v4i h[2]; };
    __device__ static Frag load(const int8_t *op, int row0, int t, int s, int lane) {
        const int row = row0 + t * 32 + (lane & 31);
        Frag f;
        f.h[0] = *reinterpret_cast<const v4i *>(op + lds_off(row, s * 4 + (lane >> 5)));
        f.h[1] = *reinterpret_cast<const v4i *>(op + lds_off(row, s * 4 + 2 + (lane >> 5)));
        return f;
    }
    __device__ static Frag load_b(const int8_t *op, int row0, int t, int s, int lane) {
        return load(op, row0, t, s, lane);
    }
    static constexpr int H = 2;   // instructions per sub-step per tile
    __device__ static void mma(Acc &c, const Frag &b, const Frag &a, int h) {
        c = __builtin_amdgcn_mfma_i32_32x32x32_i8(b.h[h], a.h[h], c, 0, 0, 0);
    }
    __device__ static Acc zero() { return Acc{0}; }
    // 32x32 result: lane holds column m = lane % 32 and, for g = 0..3, rows
    // n = 8g + 4*(lane/32) + 0..3 in registers 4g..4g+3.
    template <class F>
    __device__ static void visit(const Acc &c, int i, int j, int lane, F &&f) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
            f(i * 32 + (lane & 31), j * 32 + g * 8 + (lane >> 5) * 4,
              v4i{c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]});
    }
};

// fp8: v_mfma_f32_32x32x64_f8f6f4, FMT 0 = e4m3, 1 = e5m2 (the cbsz / blgp
// operand-format fields).  Wave tile = TI x TJ tiles of 32x32.
template <class C, int FMT = 0>
struct PolicyF8 {
    typedef C Cfg;
    static constexpr bool SUMS = false;   // u8 operand correction (PolicyU8RowB)
    static constexpr bool FLIP = false;   // u8 operands flipped to u - 128 (PolicyU8RowB)
    struct Sums {};
    template <class F> __device__ static void fixup(F &, Sums &) {}
    __device__ static void stage_hook(const int8_t *, Sums &) {}

    static constexpr int TI = C::WM / 32;
    static constexpr int TJ = C::WN / 32;
    typedef v16f Acc;
    typedef v8i Frag;
    __device__ static Frag load(const int8_t *op, int row0, int t, int s, int lane) {
        const int row = row0 + t * 32 + (lane & 31);
        const int u = s * 4 + (lane >> 5) * 2;
        const v4i lo = *reinterpret_cast<const v4i *>(op + lds_off(row, u));
        const v4i hi = *reinterpret_cast<const v4i *>(op + lds_off(row, u + 1));
        return Frag{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
    __device__ static Frag load_b(const int8_t *op, int row0, int t, int s, int lane) {
        return load(op, row0, t, s, lane);
    }
    static constexpr int H = 1;
    __device__ static void mma(Acc &c, const Frag &b, const Frag &a, int) {
        c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, FMT, FMT, 0, 0, 0, 0);
    }
    __device__ static Acc zero() { return Acc{0}; }
    // 32x32 result: lane holds column m = lane % 32 and, for g = 0..3, rows
    // n = 8g + 4*(lane/32) + 0..3 in registers 4g..4g+3.
    template <class F>
    __device__ static void visit(const Acc &c, int i, int j, int lane, F &&f) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
            f(i * 32 + (lane & 31), j * 32 + g * 8 + (lane >> 5) * 4,
              v4f{c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]});
    }
};

// ---------------------------------------------------------------------------
// Row-major B ([K, N], the RRR layout) kept in LDS as it lies in memory:
// BK = 128 k-rows of BN = 256 bytes, 16-byte unit c of row k at physical unit
// c ^ swz_t(k).  Fragments are read with ds_read_b64_tr_b8, whose 16-lane
// groups see the 8-byte values of lanes (2j, 2j+1) as row j (16 bytes) of an
// 8 x 16 byte block and return column i of it to lane i: lane i of group g
// gets 8 consecutive k of output column n0 + i, so two reads rebuild exactly
// the 16-byte, k-ascending operand that PolicyI8::load gives for A.
// swz_t(k) = 2*(k%8) + bit 4 of k gives distinct units to every set of
// (k-row, unit) pairs one 32-lane half-wave touches per read: the int8
// fragment's rows {8q..8q+7} and {8q+16..8q+23} at one unit, and the fp8
// fragment's rows {8q..8q+7} at units c and c^1.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int swz_t(int k) { return ((k & 7) << 1) | ((k >> 4) & 1); }
__device__ __forceinline__ int lds_off_t(int k, int unit) { return k * BN + ((unit ^ swz_t(k)) << 4); }

typedef int v2i_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i_t lds_v2i;

__device__ __forceinline__ v2i_t ds_read_tr8(const int8_t *p) {
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(lds_void *)p);
}

template <class C>
struct PolicyI8RowB : PolicyI8<C> {
    static_assert(C::TB == 256, "row-major B tiles are 256 columns wide");
    typedef v4i Frag;
    __device__ static Frag load_b(const int8_t *op, int row0, int t, int s, int lane) {
        // k of this lane in sub-step 0; the sub-step (+64 rows) and the high
        // half (+8 rows) leave swz_t unchanged, so they are constant offsets.
        const int kb = 16 * (lane >> 4) + ((lane & 15) >> 1);
        const int off = kb * BN + ((((row0 >> 4) + t) ^ swz_t(kb)) << 4) + ((lane & 1) << 3);
        const int8_t *q = op + off + s * 64 * BN;
        const v2i_t lo = ds_read_tr8(q);
        const v2i_t hi = ds_read_tr8(q + 8 * BN);
        return v4i{lo[0], lo[1], hi[0], hi[1]};
    }
};

// u8 x u8 RRR through the signed MFMA: fragments are flipped to u - 128
// right before the MFMA (fixup); once per stage (stage_hook) each wave sums
// the raw bytes of its slice of the freshly landed tile -- A rows
// 32*wave .. +31 (two lanes per row, ds_read_b128) and the B columns of k-rows
// 16*wave .. +15 (transposing reads: lane i of group g gets 8 k of column
// 16u + i, u = g, g+4, g+8, g+12) -- so no per-fragment sums stay live
// through the MFMA sequence.  The epilogue restores
// sum(u_a*u_b) = acc_s + 128*(rowsum + colsum) - 16384*K.
template <class C>
struct PolicyU8RowB : PolicyI8RowB<C> {
    typedef PolicyI8<C> Base;
    static constexpr bool SUMS = true;
    static constexpr bool FLIP = true;
    struct Sums {
        uint32_t ra;
        uint32_t cb[4];
    };
    template <class F>
    __device__ static void fixup(F &f, Sums &) {
#pragma unroll
        for (int t = 0; t < Base::TI; ++t) f.a[t] = u8_flip(f.a[t]);
#pragma unroll
        for (int t = 0; t < Base::TJ; ++t) f.b[t] = u8_flip(f.b[t]);
    }
    __device__ static void stage_hook(const int8_t *stage, Sums &s) {
        static_assert(C::WAVES == 8, "slices assume 8 waves");
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int row = 32 * wave + (lane >> 1);
        const int u0 = (lane & 1) * 4;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            s.ra = u8_sum16(*reinterpret_cast<const v4i *>(stage + lds_off(row, u0 + u)), s.ra);
        const int8_t *b = stage + OPER;
        const int g = lane >> 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int unit = g + 4 * q;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int k = 16 * wave + 8 * h + ((lane & 15) >> 1);
                const v2i_t v = ds_read_tr8(b + lds_off_t(k, unit) + ((lane & 1) << 3));
                s.cb[q] = __builtin_amdgcn_udot4((uint32_t)v[0], 0x01010101u, s.cb[q], false);
                s.cb[q] = __builtin_amdgcn_udot4((uint32_t)v[1], 0x01010101u, s.cb[q], false);
            }
        }
    }
};

// u8 x u8 RCR through the signed MFMA: both operands are K-contiguous rows,
// so both get PolicyU8RowB's treatment of A -- fragments flipped to u - 128
// before the MFMA, and once per stage each wave sums the raw bytes of rows
// 32*wave .. +31 of the landed A and B tiles (two lanes per row,
// ds_read_b128).  The B row sums are the output-column sums of the
// correction sum(u_a*u_b) = acc_s + 128*(rowsum + colsum) - 16384*K.
template <class C>
struct PolicyU8 : PolicyI8<C> {
    typedef PolicyI8<C> Base;
    static constexpr bool SUMS = true;
    static constexpr bool FLIP = true;
    struct Sums {
        uint32_t ra, rb;
    };
    template <class F>
    __device__ static void fixup(F &f, Sums &) {
#pragma unroll
        for (int t = 0; t < Base::TI; ++t) f.a[t] = u8_flip(f.a[t]);
#pragma unroll
        for (int t = 0; t < Base::TJ; ++t) f.b[t] = u8_flip(f.b[t]);
    }
    __device__ static void stage_hook(const int8_t *stage, Sums &s) {
        static_assert(C::WAVES == 8 && C::TB == 256, "slices assume 8 waves over 256 rows");
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int row = 32 * wave + (lane >> 1);
        const int u0 = (lane & 1) * 4;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            s.ra = u8_sum16(*reinterpret_cast<const v4i *>(stage + lds_off(row, u0 + u)), s.ra);
            s.rb = u8_sum16(*reinterpret_cast<const v4i *>(stage + C::OPER + lds_off(row, u0 + u)), s.rb);
        }
    }
};

// fp8 row-major B for the 32x32x64 policy: lane l needs the 32 k-bytes
// 64s + 32*(l/32) .. +31 of column n0 + l%32.  16-lane group g covers columns
// 16*(g%2) .. +15 and the k half g/2; four transposing reads of 8 k-rows each.
// Rows 8q + j for q = 0, 1 share swz_t, as do q = 2, 3 (unit xor 1).
template <class C, int FMT>
struct PolicyF8RowB : PolicyF8<C, FMT> {
    static_assert(C::TB == 256, "row-major B tiles are 256 columns wide");
    typedef v8i Frag;
    __device__ static Frag load_b(const int8_t *op, int row0, int t, int s, int lane) {
        const int g = lane >> 4;
        const int kb = 32 * (g >> 1) + ((lane & 15) >> 1);
        const int unit = ((row0 + t * 32) >> 4) + (g & 1);
        const int half = (lane & 1) << 3;
        const int8_t *q0 = op + kb * BN + ((unit ^ swz_t(kb)) << 4) + half + s * 64 * BN;
        const int8_t *q2 = op + (kb + 16) * BN + ((unit ^ swz_t(kb + 16)) << 4) + half + s * 64 * BN;
        const v2i_t r0 = ds_read_tr8(q0);
        const v2i_t r1 = ds_read_tr8(q0 + 8 * BN);
        const v2i_t r2 = ds_read_tr8(q2);
        const v2i_t r3 = ds_read_tr8(q2 + 8 * BN);
        return Frag{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
    }
};

template <class P>
struct Frags {
    typename P::Frag a[P::TI];
    typename P::Frag b[P::TJ];
};

template <class P>
using AccTile = typename P::Acc[P::TI][P::TJ];

template <class P>
__device__ __forceinline__ void load_frags(Frags<P> &f, const int8_t *stage, int s, int wave_m,
                                           int wave_n, int lane) {
#pragma unroll
    for (int t = 0; t < P::TJ; ++t) f.b[t] = P::load_b(stage + P::Cfg::OPER, wave_n * P::Cfg::WN, t, s, lane);
#pragma unroll
    for (int t = 0; t < P::TI; ++t) f.a[t] = P::load(stage, wave_m * P::Cfg::WM, t, s, lane);
}

// MFMAs of one sub-step over tile columns J0..J1-1.  The instruction index h
// is outermost so consecutive MFMAs never chain on the same accumulator.
template <class P, int J0, int J1>
__device__ __forceinline__ void mma_block(AccTile<P> &acc, const Frags<P> &f) {
#pragma unroll
    for (int h = 0; h < P::H; ++h)
#pragma unroll
        for (int j = J0; j < J1; ++j)
#pragma unroll
            for (int i = 0; i < P::TI; ++i) P::mma(acc[i][j], f.b[j], f.a[i], h);
}

// Buffer resource (V#) for a raw byte buffer: base, stride 0, num_records =
// `bytes` (accesses at or past it read as zero), dword3 = the gfx9-family
// raw-buffer format word.  Built wave-uniform so it lives in SGPRs.
__device__ __forceinline__ v4i make_rsrc(const void *base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    v4i r;
    r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)((a >> 32) & 0xffffu));
    r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
    r[3] = 0x00020000;
    return r;
}

// Per-thread DMA sources of one operand.  DMA instruction i (0..7) of a wave
// covers tile rows wave*64 + 8i .. +7; lane L fetches row (L/8) of that
// group at unit (L%8) ^ swz(row).
//
// Interior operand (every row of the tile is a real, evenly spaced row): swz
// of the row depends on i only through (4i & 7), so the per-lane byte offset
// is `even` (i even) or `odd` (i odd) plus the wave-uniform 8*i*ld, which
// travels in the scalar offset with the K position: 2 VGPRs per operand.
// Gathered operand (rows chosen by an index, e.g. MoE token rows): one
// per-lane offset per instruction, 8 VGPRs.
template <bool Gathered>
struct DmaOperand;

template <>
struct DmaOperand<false> {
    v4i rsrc;
    int even, odd;
    int row_stride;     // 8 * ld, bytes
};

template <>
struct DmaOperand<true> {
    v4i rsrc;
    int off[8];         // DMA_PER_WAVE used
};

// Interior operand: tile rows r0 .. r0+255 of a row-major operand with
// leading dimension ld (bytes), starting at byte `tile_off` of the buffer.
template <class C>
__device__ __forceinline__ DmaOperand<false> make_dma_interior(const int8_t *base, uint32_t bytes,
                                                               int ld, int tile_off) {
    constexpr int ROWS_PER_WAVE = C::ROWS_PER_WAVE;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    DmaOperand<false> d;
    d.rsrc = make_rsrc(base, bytes);
    d.row_stride = 8 * ld;
    const int r0 = wave * ROWS_PER_WAVE + (lane >> 3);
    const int u0 = (lane & 7) ^ swz(r0);
    d.even = tile_off + r0 * ld + u0 * 16;
    d.odd = tile_off + r0 * ld + (u0 ^ 4) * 16;
    return d;
}

// Gathered operand: `row_off(r)` gives the byte offset of tile row r.
template <class C, class RowOff>
__device__ __forceinline__ DmaOperand<true> make_dma_gathered(const int8_t *base, uint32_t bytes,
                                                              RowOff &&row_off) {
    constexpr int ROWS_PER_WAVE = C::ROWS_PER_WAVE;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    DmaOperand<true> d;
    d.rsrc = make_rsrc(base, bytes);
#pragma unroll
    for (int i = 0; i < C::DMA_PER_WAVE; ++i) {
        const int r = wave * ROWS_PER_WAVE + i * 8 + (lane >> 3);
        d.off[i] = row_off(r) + ((lane & 7) ^ swz(r)) * 16;
    }
    return d;
}

// One LDS-DMA transfer: 16 bytes per lane from rsrc[voff + soff] into LDS at
// `lds_dst + 16 * lane` (lds_dst wave-uniform, passed through M0).  Issued as
// inline asm so the compiler's wait-count pass does not treat consecutive
// DMAs into one buffer as dependent (it would wait vmcnt(0) before each);
// completion is awaited explicitly by wait_dma() before the stage barrier.
// The M0 value is the low 32 bits of the generic address: in the LDS
// aperture those are the LDS byte offset, and taking them directly avoids
// the null-pointer select of an address-space cast, so the whole destination
// computation stays in scalar registers (callers pass a wave-uniform
// pointer built from a readfirstlane wave index).
__device__ __forceinline__ void dma16(const v4i &rsrc, int voff, int soff, const int8_t *lds_dst) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(lds_dst));
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Wait until at most N of this wave's vector-memory operations (DMAs
// included) are outstanding; they complete in issue order.
template <int N>
__device__ __forceinline__ void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// Last rows of M run by a separate last-rows launch instead of a row of
// 256-row tiles (N % 16 == 0): M % 256 in [1, limit] (all of M when
// M <= limit: no tiles at all), when that row of tiles would start another
// round of tiles on the 256 CUs (it costs nothing extra when it fits the
// idle CUs of the last round).  Returns the number of last rows, or 0.
// Column fragments (16 columns each) per workgroup of a last-rows pass: the
// widest of 4, 2, 1 that divides N / 16 and still leaves at least 192
// workgroups (3/4 of the CUs).  Every workgroup reads the pass's A rows once,
// so wider groups cut the A traffic, but fewer than ~a CU's worth of
// workgroups leave CUs idle (int8, K = 4096, M = 32 / 128: N = 4096
// 7.2 / 11.8 us with 16 columns against 7.8 / 13.2 with 32; N = 14336
// 19.2 / 39.4 us with 16 columns against 14.5 / 20.0 with 64).
// `blocks`: row blocks of the pass (gridDim.y), which multiply the
// workgroup count.
inline int last_rows_col_frags(int N, int blocks = 1) {
    for (int nb = 4; nb > 1; nb /= 2)
        if (N % (16 * nb) == 0 && N / (16 * nb) * blocks >= 192) return nb;
    return 1;
}

// Row blocks of a last-rows pass of 33-128 rows when the rule above gives
// 16-column workgroups (N below 6144), which would each stage all the rows:
// blocks of 32 rows, or of 64 rows for more than 64 rows when N > 2048, the
// column width by the rule over the blocks.  Measured at K = 4096 (graph
// replay, rotated weights): N = 4096, M = 65 / 100 / 128 in 64-row blocks of
// 32 columns 8.8 / 9.1 / 9.5 us, in 32-row blocks of 64 columns 9.6 / 9.9 /
// 10.3; N = 2048 in 32-row blocks of 32 columns 6.4 / 6.4 / 6.5 us, in
// 64-row blocks of 16 columns 6.9; 33-64 rows as two 32-row blocks: N =
// 4096 / 2048, M = 48 7.8 / 5.8 us against 8.5 / 6.8 as one block.
inline void last_rows_blocks(int rem, int N, int &rf, int &blocks, int &nb) {
    rf = rem > 64 && N > 2048 ? 4 : 2;
    blocks = (rem + 16 * rf - 1) / (16 * rf);
    nb = last_rows_col_frags(N, blocks);
}

inline int last_rows_pass(int M, int N, int limit) {
    if (N <= 0 || N % 16 != 0 || M <= 0) return 0;
    const int rem = M % 256;
    if (rem == 0 || rem > limit) return 0;
    const int64_t tn = (N + 255) / 256, main_tiles = (int64_t)(M - rem) / 256 * tn;
    if (main_tiles > 0 && (main_tiles + tn + 255) / 256 == (main_tiles + 255) / 256) return 0;
    return rem;
}

template <class C>
__device__ __forceinline__ void dma_operand(int8_t *dst, const DmaOperand<false> &d, int kbyte) {
    constexpr int ROWS_PER_WAVE = C::ROWS_PER_WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < C::DMA_PER_WAVE; ++i) {
        const int soff = __builtin_amdgcn_readfirstlane(kbyte + i * d.row_stride);
        dma16(d.rsrc, (i & 1) ? d.odd : d.even, soff, dst + (wave * ROWS_PER_WAVE + i * 8) * BK);
    }
}

template <class C>
__device__ __forceinline__ void dma_operand(int8_t *dst, const DmaOperand<true> &d, int kbyte) {
    constexpr int ROWS_PER_WAVE = C::ROWS_PER_WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int soff = __builtin_amdgcn_readfirstlane(kbyte);
#pragma unroll
    for (int i = 0; i < C::DMA_PER_WAVE; ++i) dma16(d.rsrc, d.off[i], soff, dst + (wave * ROWS_PER_WAVE + i * 8) * BK);
}

// Row-major B operand ([K, N], leading dimension ld): one DMA instruction
// writes 4 k-rows of 256 bytes; lane L lands in row L/16 at physical unit
// L%16 and so fetches logical unit (L%16) ^ swz_t(row).  For 8 waves a wave
// owns 16 k-rows (4 instructions) and swz_t of its rows depends on the
// instruction only through its parity, so as for the interior operand the
// per-lane offset is `even` or `odd`, and the K position plus 4*i*ld travel
// in the scalar offset.
struct DmaOperandRowB {
    v4i rsrc;
    int even, odd;
    int ld;
};

template <class C>
__device__ __forceinline__ DmaOperandRowB make_dma_row_b(const int8_t *base, uint32_t bytes, int ld,
                                                         int n_base) {
    static_assert(BK / C::WAVES == 16, "row-major B DMA assumes 16 k-rows per wave");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    DmaOperandRowB d;
    d.rsrc = make_rsrc(base, bytes);
    d.ld = ld;
    const int r0 = wave * 16 + (lane >> 4);
    const int p = lane & 15;
    d.even = n_base + r0 * ld + ((p ^ swz_t(r0)) << 4);
    d.odd = n_base + r0 * ld + ((p ^ swz_t(r0 + 4)) << 4);
    return d;
}

template <class C>
__device__ __forceinline__ void dma_operand(int8_t *dst, const DmaOperandRowB &d, int kbyte) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int soff = __builtin_amdgcn_readfirstlane((kbyte + 4 * i) * d.ld);
        dma16(d.rsrc, (i & 1) ? d.odd : d.even, soff, dst + (wave * 16 + 4 * i) * BN);
    }
}

struct DmaRowsRrr {
    DmaOperand<false> a;
    DmaOperandRowB b;
};

template <bool GA, bool GB>
struct DmaRows {
    DmaOperand<GA> a;
    DmaOperand<GB> b;
};

template <class C, class D>
__device__ __forceinline__ void dma_stage(int8_t *stage, const D &d, int kbyte) {
    dma_operand<C>(stage, d.a, kbyte);
    dma_operand<C>(stage + C::OPER, d.b, kbyte);
}

// One stage: compute from `cur`, stream the next stage into `nxt` (if any).
template <class P, class D>
__device__ __forceinline__ void stage_step(AccTile<P> &acc, Frags<P> &f0, Frags<P> &f1,
                                           const int8_t *cur, int8_t *nxt, const D &d, int next_k,
                                           bool has_next, int wave_m, int wave_n, int lane,
                                           typename P::Sums &sums) {
    typedef typename P::Cfg C;
    if (has_next) dma_stage<C>(nxt, d, next_k);
    load_frags<P>(f0, cur, 0, wave_m, wave_n, lane);
    if constexpr (P::FLIP) P::fixup(f0, sums);
    mma_block<P, 0, P::TJ>(acc, f0);
    // u8: the flip's temporaries leave no room for both fragment sets, so the
    // second sub-step's reads are not hoisted over the first's MFMAs.
    if constexpr (P::FLIP) __builtin_amdgcn_sched_barrier(0);
    load_frags<P>(f1, cur, 1, wave_m, wave_n, lane);
    if constexpr (P::FLIP) P::fixup(f1, sums);
    mma_block<P, 0, P::TJ>(acc, f1);
    // `cur` stays valid until the barrier below; the fragments are dead here.
    if constexpr (P::SUMS) P::stage_hook(cur, sums);
    wait_dma();        // this wave's DMA into `nxt` has landed
    __syncthreads();   // ... and every wave's; every wave is done reading `cur`
}

// Full K loop for one 256x256 tile.  s0 / s1 are the two stage buffers
// (each 2 * OPER bytes: A then B).  Ends with a barrier.
template <class P, class D>
__device__ __forceinline__ void mainloop(int8_t *s0, int8_t *s1, const D &d, int K, AccTile<P> &acc,
                                         typename P::Sums &sums) {
    typedef typename P::Cfg C;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wave_m = wave / C::WAVES_N, wave_n = wave % C::WAVES_N;
#pragma unroll
    for (int i = 0; i < P::TI; ++i)
#pragma unroll
        for (int j = 0; j < P::TJ; ++j) acc[i][j] = P::zero();

    const int KT = K / BK;
    Frags<P> f0, f1;
    dma_stage<C>(s0, d, 0);
    wait_dma();
    __syncthreads();
    int kt = 0;
    for (; kt + 2 <= KT; kt += 2) {
        stage_step<P>(acc, f0, f1, s0, s1, d, (kt + 1) * BK, true, wave_m, wave_n, lane, sums);
        stage_step<P>(acc, f0, f1, s1, s0, d, (kt + 2) * BK, kt + 2 < KT, wave_m, wave_n, lane, sums);
    }
    if (kt < KT) stage_step<P>(acc, f0, f1, s0, s1, d, 0, false, wave_m, wave_n, lane, sums);
}

template <class P, class D>
__device__ __forceinline__ void mainloop(int8_t *s0, int8_t *s1, const D &d, int K, AccTile<P> &acc) {
    static_assert(!P::SUMS, "this policy needs its operand sums");
    typename P::Sums none;
    mainloop<P>(s0, s1, d, K, acc, none);
}

// The DMA and barrier sequence of mainloop() without fragment reads or
// MFMAs, for a wave whose output rows are all padding: it still moves its
// share of every stage and meets every barrier of the waves that compute.
template <class C, class D>
__device__ __forceinline__ void mainloop_dma_only(int8_t *s0, int8_t *s1, const D &d, int K) {
    const int KT = K / BK;
    dma_stage<C>(s0, d, 0);
    wait_dma();
    __syncthreads();
    int kt = 0;
    for (; kt + 2 <= KT; kt += 2) {
        dma_stage<C>(s1, d, (kt + 1) * BK);
        wait_dma();
        __syncthreads();
        if (kt + 2 < KT) dma_stage<C>(s0, d, (kt + 2) * BK);
        wait_dma();
        __syncthreads();
    }
    if (kt < KT) {
        wait_dma();
        __syncthreads();
    }
}

// W8A8 bf16 epilogue for the int8 16x16 policy, staged through LDS so each
// output row segment of the wave tile (WN bf16 = 128 bytes for WN = 64) is
// written with full-line 16-byte stores.
//   sam[i]   dequant scale of this lane's row in 16-row tile i
//   post[i]  optional second row factor (1 multiply after the dequant), only
//            read when HasPost
//   swv[j]   the 4 column scales of this lane's quad in 16-column tile j
//   row_dst(r) destination of wave-tile row r (0..WM-1) at the wave's first
//            column, or nullptr to skip the row
// `scratch` holds WM*WN*2 bytes private to this wave; LDS must be free (the
// mainloop ends with a barrier).  Products are rounded in the order
// ((sam * sw) * acc) [* post], then packed with v_cvt_pk_bf16_f32.
//   ncols    valid columns of the wave tile (a multiple of 8; units at or
//            past it are not stored: the N edge of a partial tile)
template <class P, bool HasPost, class RowDst>
__device__ __forceinline__ void store_w8a8_bf16_staged(const AccTile<P> &acc, int8_t *scratch,
                                                       const float (&sam)[P::TI],
                                                       const float (&post)[P::TI],
                                                       const v4f (&swv)[P::TJ], RowDst &&row_dst,
                                                       int ncols = P::Cfg::WN) {
    typedef typename P::Cfg C;
    static_assert(C::WN * 2 == 128, "staged store assumes 128-byte wave-tile rows");
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < P::TI; ++i)
#pragma unroll
        for (int j = 0; j < P::TJ; ++j) {
            float y[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                y[r] = (sam[i] * swv[j][r]) * (float)acc[i][j][r];
                if constexpr (HasPost) y[r] = y[r] * post[i];
            }
            const int row = i * 16 + (lane & 15);
            const int col = j * 16 + (lane >> 4) * 4;              // bf16 column
            const int unit = col >> 3, half = (col >> 2) & 1;
            v2i w;
            w[0] = (int)f32x2_to_bf16x2(y[0], y[1]);
            w[1] = (int)f32x2_to_bf16x2(y[2], y[3]);
            *reinterpret_cast<v2i *>(scratch + row * 128 + ((unit ^ (row & 7)) << 4) + half * 8) = w;
        }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int q = 0; q < C::WM / 8; ++q) {
        const int row = q * 8 + (lane >> 3), u = lane & 7;
        uint16_t *dst = row_dst(row);
        if (dst == nullptr || u * 8 >= ncols) continue;
        const v4i v = *reinterpret_cast<const v4i *>(scratch + row * 128 + ((u ^ (row & 7)) << 4));
        // Non-temporal: the 32 MiB output of a 4096^2 tile grid streams past
        // the caches instead of evicting the operands still being read.
        __builtin_nontemporal_store(v, reinterpret_cast<v4i *>(dst + u * 8));
    }
}

// 1-byte outputs of any policy whose wave tile is WN = 64 columns, staged in
// LDS so each 64-byte row of the wave tile is written with 16-byte stores.
//   pack(r, c, quad)  4 output bytes of wave-tile row r, columns c..c+3
//   row_dst(r)        destination of wave-tile row r at the wave's first column
//                     (nullptr: row not stored)
//   ncols             valid columns of the wave tile (a multiple of 16 bytes)
// `scratch`: WM * WN bytes private to this wave.  16-byte unit u of row r
// sits at unit u ^ ((r >> 2) & 3), so the 16 rows of one 4-byte write
// instruction fall in distinct banks.
template <class P, class Pack, class RowDst>
__device__ __forceinline__ void store_u8x4_staged(const AccTile<P> &acc, int8_t *scratch, Pack &&pack,
                                                  RowDst &&row_dst, int ncols = P::Cfg::WN) {
    typedef typename P::Cfg C;
    static_assert(C::WN == 64, "staged byte store assumes 64-byte wave-tile rows");
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < P::TI; ++i)
#pragma unroll
        for (int j = 0; j < P::TJ; ++j)
            P::visit(acc[i][j], i, j, lane, [&](int r, int c, const auto &v) {
                const int unit = (c >> 4) ^ ((r >> 2) & 3);
                *reinterpret_cast<uint32_t *>(scratch + r * 64 + (unit << 4) + (c & 15)) = pack(r, c, v);
            });
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int q = 0; q < C::WM / 16; ++q) {
        const int r = q * 16 + (lane >> 2), u = lane & 3;
        const v4i v = *reinterpret_cast<const v4i *>(scratch + r * 64 + ((u ^ ((r >> 2) & 3)) << 4));
        auto *dst = row_dst(r);
        if (dst != nullptr && u * 16 < ncols) __builtin_nontemporal_store(v, reinterpret_cast<v4i *>(dst + u * 16));
    }
}

// 32-bit outputs of a policy whose wave tile is WN = 64 columns (256-byte
// rows): each quad (4 columns of one row) is packed to 16 bytes by
// pack(r, c, quad) and the wave tile staged in LDS in two halves of WM / 2
// rows (`scratch`: WM / 2 * 256 bytes private to this wave; unit u of row r
// at unit u ^ (r & 15)), each half's rows written as 16-byte units, four
// rows of 256 bytes per store instruction.  row_dst(r) gives row r's
// destination (nullptr: skip); ncols: valid columns (a multiple of 4).
template <class P, class Pack, class RowDst>
__device__ __forceinline__ void store_x32x4_staged(const AccTile<P> &acc, int8_t *scratch, Pack &&pack,
                                                   RowDst &&row_dst, int ncols = P::Cfg::WN) {
    typedef typename P::Cfg C;
    static_assert(C::WN == 64 && P::TI % 2 == 0, "staged 32-bit store assumes 256-byte wave-tile rows");
    constexpr int HALF = C::WM / 2;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int i = h * (P::TI / 2); i < (h + 1) * (P::TI / 2); ++i)
#pragma unroll
            for (int j = 0; j < P::TJ; ++j)
                P::visit(acc[i][j], i, j, lane, [&](int r, int c, const auto &v) {
                    const int rl = r - h * HALF;
                    const int unit = (c >> 2) ^ (rl & 15);
                    *reinterpret_cast<v4i *>(scratch + rl * 256 + (unit << 4)) = pack(r, c, v);
                });
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int q = 0; q < HALF / 4; ++q) {
            const int rl = q * 4 + (lane >> 4), u = lane & 15;
            const v4i v = *reinterpret_cast<const v4i *>(scratch + rl * 256 + ((u ^ (rl & 15)) << 4));
            auto *dst = row_dst(h * HALF + rl);   // 32-bit elements
            if (dst != nullptr && u * 4 < ncols) __builtin_nontemporal_store(v, reinterpret_cast<v4i *>(dst + u * 4));
        }
        // the second half reuses the scratch rows
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// 64-bit outputs of the int8 16x16 policy (WN = 64 columns, 512-byte rows):
// each quad is packed to 32 bytes by pack(r, c, quad) -> {lo, hi} (columns
// c, c+1 and c+2, c+3) and the wave tile staged in LDS in four quarters of
// WM / 4 rows (`scratch`: WM / 4 * 512 bytes private to this wave; 16-byte
// unit u of row r at unit u ^ (r & 15)), two 512-byte rows per store
// instruction.  row_dst(r): row r's destination (nullptr: skip); ncols:
// valid columns (a multiple of 2).
struct Quad64 { v4i lo, hi; };

template <class P, class Pack, class RowDst>
__device__ __forceinline__ void store_x64x4_staged(const AccTile<P> &acc, int8_t *scratch, Pack &&pack,
                                                   RowDst &&row_dst, int ncols = P::Cfg::WN) {
    typedef typename P::Cfg C;
    static_assert(C::WN == 64 && P::TI % 4 == 0, "staged 64-bit store assumes 512-byte wave-tile rows");
    constexpr int QR = C::WM / 4;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
#pragma unroll
        for (int i = h * (P::TI / 4); i < (h + 1) * (P::TI / 4); ++i)
#pragma unroll
            for (int j = 0; j < P::TJ; ++j)
                P::visit(acc[i][j], i, j, lane, [&](int r, int c, const auto &v) {
                    const int rl = r - h * QR;
                    const Quad64 q = pack(r, c, v);
                    const int u0 = (c >> 1) ^ (rl & 15), u1 = ((c >> 1) + 1) ^ (rl & 15);
                    *reinterpret_cast<v4i *>(scratch + rl * 512 + (u0 << 4)) = q.lo;
                    *reinterpret_cast<v4i *>(scratch + rl * 512 + (u1 << 4)) = q.hi;
                });
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int q = 0; q < QR / 2; ++q) {
            const int rl = q * 2 + (lane >> 5), u = lane & 31;
            const v4i v = *reinterpret_cast<const v4i *>(scratch + rl * 512 + ((u ^ (rl & 15)) << 4));
            auto *dst = row_dst(h * QR + rl);   // 64-bit elements
            if (dst != nullptr && u * 2 < ncols) __builtin_nontemporal_store(v, reinterpret_cast<v4i *>(dst + u * 2));
        }
        // the next quarter reuses the scratch rows
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// 16-bit outputs of any policy whose wave tile is WN = 64 columns: each quad
// (4 columns of one row) is packed to 4 halves by pack(r, c, quad) (8 bytes)
// and staged in LDS; rows (128 bytes) are then written as 16-byte units,
// row_dst(r) giving each row's destination (nullptr: skip the row).
// `scratch`: WM * 128 bytes private to this wave; unit u of row r sits at
// unit u ^ (r & 7).
// ncols: valid columns of the wave tile (a multiple of 8), units past it are
// not stored.
template <class P, class Pack, class RowDst>
__device__ __forceinline__ void store_bf16x4_staged(const AccTile<P> &acc, int8_t *scratch, Pack &&pack,
                                                    RowDst &&row_dst, int ncols = P::Cfg::WN) {
    typedef typename P::Cfg C;
    static_assert(C::WN == 64, "staged bf16 store assumes 128-byte wave-tile rows");
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < P::TI; ++i)
#pragma unroll
        for (int j = 0; j < P::TJ; ++j)
            P::visit(acc[i][j], i, j, lane, [&](int r, int c, const auto &v) {
                const int unit = (c >> 3) ^ (r & 7);
                *reinterpret_cast<v2i *>(scratch + r * 128 + (unit << 4) + ((c & 7) << 1)) = pack(r, c, v);
            });
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int q = 0; q < C::WM / 8; ++q) {
        const int r = q * 8 + (lane >> 3), u = lane & 7;
        const v4i v = *reinterpret_cast<const v4i *>(scratch + r * 128 + ((u ^ (r & 7)) << 4));
        uint16_t *dst = row_dst(r);   // nullptr: row not stored
        if (dst != nullptr && u * 8 < ncols) __builtin_nontemporal_store(v, reinterpret_cast<v4i *>(dst + u * 8));
    }
}

// Visit this thread's accumulators: f(m_local, n0_local, quad) with quad the
// values of columns n0..n0+3 of row m.
template <class P, class F>
__device__ __forceinline__ void for_each_quad(const AccTile<P> &acc, F &&f) {
    typedef typename P::Cfg C;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave / C::WAVES_N) * C::WM, wn = (wave % C::WAVES_N) * C::WN;
#pragma unroll
    for (int i = 0; i < P::TI; ++i)
#pragma unroll
        for (int j = 0; j < P::TJ; ++j)
            P::visit(acc[i][j], i, j, lane, [&](int m, int n0, auto q) { f(wm + m, wn + n0, q); });
}

}  // namespace mfma2
}  // namespace bk
