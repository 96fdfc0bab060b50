// moe_grouped.hip -- grouped MoE expert GEMMs for gfx950, one GEMM launch
// over all experts:
//   int8 x int8 with the W8A8 dequant epilogue to bf16 (new SKU), and
//   bf16 x bf16 / f16 x f16 with f32 accumulation (the reference's moe_wmma).
//
// Routing contract of the reference MoE path
// (crates/baracuda-kernels-sys/kernels/moe/moe_wmma.cu:121-175,
//  crates/baracuda-kernels-sys/kernels/include/baracuda_moe.cuh:827-944,1121-1162):
//   sorted_token_ids[size_m]  pair ids (token*topk + slot) grouped by expert
//   expert_ids[size_m]        expert of each sorted position
//   expert_counts[E], expert_offsets[E+1]   caller-provided, filled here
//   input row of pair p       = sorted_token_ids[p] / topk   (topk_weights == NULL)
//                             = sorted_token_ids[p]          (topk_weights != NULL)
//   output row of pair p      = sorted_token_ids[p]
//   int8:      out[row, n] = bf16( ((sa[in_row] * sw[e*N + n]) * acc) [* topk_weights[row]] )
//   bf16/f16:  out[row, n] = T( acc [* topk_weights[row]] )   (baracuda_moe.cuh:929-941)
//   int8, i32: out[row, n] = acc (int32), the accumulator the W8A8 SKU
//              dequantizes: same kernel, same mainloop, no epilogue arithmetic
//
// Differences by design: expert offsets are computed by one workgroup with
// LDS counters (no global atomics, no memset: graph-capturable), and the GEMM
// is one launch whose workgroups walk the ragged per-expert tile list.
#include "gemm_mfma.hpp"
#include "gemm_mfma2.hpp"

namespace bk {
namespace {

using namespace mfma;

constexpr int kMaxExperts = 1024;

// expert_counts / expert_offsets from expert_ids (one workgroup, 1024 threads).
// Up to 64 experts each wave counts 64 ids at a time with one ballot per
// expert, lane e keeping expert e's running count, and adds its counts to
// LDS once; more experts fall back to one LDS atomic per id.  Ids outside
// [0, num_experts) are not counted.
__global__ __launch_bounds__(1024) void moe_offsets_kernel(const int32_t *__restrict__ expert_ids,
                                                           int32_t size_m, int32_t num_experts,
                                                           int32_t *__restrict__ counts,
                                                           int32_t *__restrict__ offsets) {
    __shared__ int32_t cnt[kMaxExperts];
    for (int e = threadIdx.x; e < num_experts; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    if (num_experts <= 64) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
        int mine = 0;   // count of expert `lane`
        // Each wave takes 8 ids per lane per pass, all loads issued before the
        // first ballot so one memory round trip covers 512 ids.
        constexpr int V = 8;
        for (int base = wave * 64 * V; base < size_m; base += waves * 64 * V) {
            int e[V];
#pragma unroll
            for (int v = 0; v < V; ++v) {
                const int i = base + v * 64 + lane;
                e[v] = i < size_m ? expert_ids[i] : -1;
            }
#pragma unroll
            for (int v = 0; v < V; ++v)
                for (int x = 0; x < num_experts; ++x) {
                    const int c = __popcll(__ballot(e[v] == x));
                    if (lane == x) mine += c;
                }
        }
        if (lane < num_experts && mine) atomicAdd(&cnt[lane], mine);
    } else {
        for (int i = threadIdx.x; i < size_m; i += blockDim.x) {
            const int e = expert_ids[i];
            if (e >= 0 && e < num_experts) atomicAdd(&cnt[e], 1);
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        offsets[0] = 0;
        for (int e = 0; e < num_experts; ++e) {
            counts[e] = cnt[e];
            run += cnt[e];
            offsets[e + 1] = run;
        }
    }
}

// Operand kinds: int8 (W8A8 epilogue), bf16, f16 (16-bit float elements),
// int8 with the int32 accumulator as output.
enum MoeKind : int { MOE_S8 = 0, MOE_BF16 = 1, MOE_F16 = 2, MOE_S8_I32 = 3 };

template <int KIND> struct MoeElem;
template <> struct MoeElem<MOE_S8> { static constexpr Elem E = Elem::S8; static constexpr int SIZE = 1; };
template <> struct MoeElem<MOE_BF16> { static constexpr Elem E = Elem::BF16; static constexpr int SIZE = 2; };
template <> struct MoeElem<MOE_F16> { static constexpr Elem E = Elem::F16; static constexpr int SIZE = 2; };
template <> struct MoeElem<MOE_S8_I32> { static constexpr Elem E = Elem::S8; static constexpr int SIZE = 1; };

struct MoeArgs {
    const int8_t *x;            // [tokens, K] elements (bytes addressed)
    const int8_t *w;            // [E, N, K]
    const int32_t *sorted_ids;  // [size_m]
    const int32_t *offsets;     // [E+1]
    const float *topk_w;        // [size_m] or nullptr
    const float *sa;            // [tokens]   (int8 only)
    const float *sw;            // [E, N]     (int8 only)
    void *out;                  // [size_m, N] bf16 / f16 (int32 for MOE_S8_I32)
    int E, topk, size_m, N, K;  // K in elements
    // Decode launches only (size_m <= 64): the ids, and the counts / offsets
    // they write in place of moe_offsets_kernel.
    const int32_t *expert_ids = nullptr;   // [size_m], sorted
    int32_t *counts = nullptr;             // [E]
};

// Decode launches (size_m <= 64, no offsets kernel): expert e's first
// sorted position and row count from the ids, one ballot each in wave 0
// (ids outside [0, E) are counted nowhere, as in moe_offsets_kernel); the
// workgroups of column group 0 write the counts and offsets that kernel
// would.  Workgroup-uniform results; contains a barrier.
__device__ __forceinline__ void moe_decode_rows(const MoeArgs &p, int e, int &o0, int &rows) {
    __shared__ int s_rows[2];
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const int id = lane < p.size_m ? p.expert_ids[lane] : -1;
        const int before = __popcll(__ballot(id >= 0 && id < e));
        const int mine = __popcll(__ballot(id == e));
        if (lane == 0) {
            s_rows[0] = before;
            s_rows[1] = mine;
            if (blockIdx.x == 0 && blockIdx.z == 0) {
                int32_t *off = const_cast<int32_t *>(p.offsets);
                p.counts[e] = mine;
                off[e + 1] = before + mine;
                if (e == 0) off[0] = 0;
            }
        }
    }
    __syncthreads();
    o0 = s_rows[0];
    rows = s_rows[1];
}

// The E+1 offsets, clamped to size_m, loaded in one parallel step into LDS.
__device__ __forceinline__ void moe_load_offsets(const MoeArgs &p, int32_t *s_off) {
    for (int i = threadIdx.x; i <= p.E; i += blockDim.x) s_off[i] = min(p.offsets[i], p.size_m);
    __syncthreads();
}

// Ragged tile list: slot -> (expert, first pair of the tile, rows in it),
// walked by every thread from the offsets in LDS (workgroup-uniform result);
// false past the last tile.
__device__ __forceinline__ bool moe_find(const MoeArgs &p, const int32_t *s_off, int slot, int &e,
                                         int &seg0, int &rows_out) {
    for (e = 0; e < p.E; ++e) {
        const int o0 = s_off[e], o1 = s_off[e + 1];
        const int rows = o1 > o0 ? o1 - o0 : 0;
        const int tiles = (rows + 255) / 256;
        if (slot < tiles) {
            seg0 = o0 + slot * 256;
            rows_out = min(256, rows - slot * 256);
            return true;
        }
        slot -= tiles;
    }
    return false;
}

__device__ __forceinline__ bool moe_tile(const MoeArgs &p, int32_t *s_off, int slot, int &e,
                                         int &seg0, int &rows_out) {
    moe_load_offsets(p, s_off);
    return moe_find(p, s_off, slot, e, seg0, rows_out);
}

// W8A8 epilogue of one group of 4 columns of tile row ml.
__device__ __forceinline__ void moe_store(const MoeArgs &p, const int32_t *rows_tok, int seg_rows,
                                          int in_div, const float *swe, int ml, int n0,
                                          const v4i &v) {
    if (ml >= seg_rows || n0 >= p.N) return;
    const int tok = rows_tok[ml];
    const float sam = p.sa[tok / in_div];
    const int count = p.N - n0 < 4 ? p.N - n0 : 4;
    float y[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = r < count ? (sam * swe[n0 + r]) * (float)v[r] : 0.0f;
    if (p.topk_w) {
        const float tw = p.topk_w[tok];
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = y[r] * tw;
    }
    store4_bf16(static_cast<uint16_t *>(p.out) + (int64_t)tok * p.N + n0, y, count == 4 && (p.N % 4 == 0),
                count);
}

// int32 accumulator out, one group of 4 columns of tile row ml.
__device__ __forceinline__ void moe_store_i32(const MoeArgs &p, const int32_t *rows_tok, int seg_rows, int ml,
                                              int n0, const v4i &v) {
    if (ml >= seg_rows || n0 >= p.N) return;
    int32_t *d = static_cast<int32_t *>(p.out) + (int64_t)rows_tok[ml] * p.N + n0;
    const int count = p.N - n0 < 4 ? p.N - n0 : 4;
    if (count == 4 && (reinterpret_cast<uintptr_t>(d) & 15u) == 0) {
        *reinterpret_cast<v4i *>(d) = v;
    } else {
        for (int r = 0; r < count; ++r) d[r] = v[r];
    }
}

// bf16 / f16 epilogue of one group of 4 columns: out = T(acc [* topk_w]).
template <int KIND, class AccV>
__device__ __forceinline__ void moe_store_h(const MoeArgs &p, const int32_t *rows_tok, int seg_rows,
                                            int ml, int n0, const AccV &v) {
    if (ml >= seg_rows || n0 >= p.N) return;
    const int tok = rows_tok[ml];
    const int count = p.N - n0 < 4 ? p.N - n0 : 4;
    const float tw = p.topk_w ? p.topk_w[tok] : 1.0f;
    uint16_t h[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float y = p.topk_w ? v[r] * tw : v[r];
        h[r] = KIND == MOE_BF16 ? f32_to_bf16_rne(y) : f32_to_f16_rne(y);
    }
    uint16_t *d = static_cast<uint16_t *>(p.out) + (int64_t)tok * p.N + n0;
    if (count == 4 && (reinterpret_cast<uintptr_t>(d) & 7u) == 0) {
        *reinterpret_cast<v2i *>(d) = v2i{(int)((uint32_t)h[0] | ((uint32_t)h[1] << 16)),
                                          (int)((uint32_t)h[2] | ((uint32_t)h[3] << 16))};
    } else {
        for (int r = 0; r < count; ++r) d[r] = h[r];
    }
}

// General path (K tail / unaligned / N not a multiple of 256).
template <int KIND>
__global__ __launch_bounds__(NT, 1) void moe_grouped_kernel(MoeArgs p) {
    constexpr int ES = MoeElem<KIND>::SIZE;
    __shared__ __attribute__((aligned(16))) int8_t lds[4 * LDS_TILE];
    __shared__ int32_t s_rows_tok[BM];
    __shared__ int32_t s_off[kMaxExperts + 1];
    int e, seg0, seg_rows;
    if (!moe_tile(p, s_off, blockIdx.x, e, seg0, seg_rows)) return;   // whole workgroup exits
    const int n_base = blockIdx.y * BN;
    const int tid = threadIdx.x;
    for (int r = tid; r < BM; r += NT) s_rows_tok[r] = p.sorted_ids[seg0 + min(r, seg_rows - 1)];
    __syncthreads();
    const int in_div = p.topk_w ? 1 : p.topk;
    const int64_t kb = (int64_t)p.K * ES;   // row length in bytes
    const int8_t *we = p.w + (int64_t)e * p.N * kb;
    RowSet as, bs;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int r = i * LOAD_ROWS + (tid >> 3);
        as.ptr[i] = p.x + (int64_t)(s_rows_tok[r] / in_div) * kb;
        bs.ptr[i] = we + (int64_t)min(n_base + r, p.N - 1) * kb;
    }
    typename AccT<MoeElem<KIND>::E>::type acc[TM][TN];
    mainloop<MoeElem<KIND>::E, true>(lds, as, bs, (int)kb, acc);
    if constexpr (KIND == MOE_S8) {
        const float *swe = p.sw + (int64_t)e * p.N;
        for_each_fragment(acc, [&](int ml, int nl, const v4i &v) {
            moe_store(p, s_rows_tok, seg_rows, in_div, swe, ml, n_base + nl, v);
        });
    } else if constexpr (KIND == MOE_S8_I32) {
        for_each_fragment(acc, [&](int ml, int nl, const v4i &v) {
            moe_store_i32(p, s_rows_tok, seg_rows, ml, n_base + nl, v);
        });
    } else {
        for_each_fragment(acc, [&](int ml, int nl, const v4f &v) {
            moe_store_h<KIND>(p, s_rows_tok, seg_rows, ml, n_base + nl, v);
        });
    }
}

// Fast path: K % 128 == 0, N % 256 == 0, 16-byte aligned operands.  A rows
// are gathered per tile row (token rows of the expert's segment), B is the
// expert's weight slab.
typedef mfma2::Cfg<2, 4> DmaCfg;

// Workgroup id -> tile of the compact ragged list.  The list holds
// T = S * n_tiles tiles (S = sum_e ceil(cnt_e / 256) m-tiles, from the
// offsets in LDS), in blocks of kMoeNBlock n-tiles: block b holds every
// (slot, n-tile) pair of its n-tiles, n-tile fastest, so that the tiles an
// XCD runs together share A panels (4 n-tiles per slot) as well as the
// expert's weight panels (consecutive slots of one expert).  Workgroups
// are dispatched round-robin over the 8 XCDs; the id is regrouped so each
// XCD owns a contiguous range of the list.  Ids past the list exit (the
// grid is sized for the largest possible S).  Config 5, one box, four
// alternating passes: blocks of 1 / 2 / 3 / 4 / 8 / 16 n-tiles 536–539 /
// 528–542 / 520–528 / 512–526 / 517–525 / 529–539 µs (1 is the plain
// slot-fastest order); against a regroup over the largest grid, whose
// surplus slots exited inside every XCD's range, the compact list alone
// measured 567 against 577 µs.
constexpr int kMoeNBlock = 4;

// Reordered tail of each XCD's range (see moe_dma_coords).  Config 5, two
// boxes, six alternating passes each: windows of 16 / 32 / 48 / 64 / 128
// positions 494 / 494 / 496 / 498 / 522 against 510 µs without (the
// 128-position window reaches back into earlier n-blocks, whose weight
// panels have left the caches).
constexpr int kMoeTail = 32;

// List position -> (slot, n-tile) in the n-block order.
__device__ __forceinline__ void moe_list_tile(int r, int S, int n_tiles, int &slot, int &ntile) {
    const int b = r / (S * kMoeNBlock);
    const int bw = min(kMoeNBlock, n_tiles - b * kMoeNBlock);   // the last block may be narrower
    const int i = r - b * S * kMoeNBlock;
    slot = i / bw;
    ntile = b * kMoeNBlock + i % bw;
}

__device__ __forceinline__ bool moe_dma_coords(const MoeArgs &p, const int32_t *s_off, int pid,
                                               int n_tiles, int &slot, int &ntile, int *s_tail) {
    constexpr int XCDS = 8;
    int S = 0;
    for (int e = 0; e < p.E; ++e) {
        const int rows = s_off[e + 1] > s_off[e] ? s_off[e + 1] - s_off[e] : 0;
        S += (rows + 255) / 256;
    }
    const int T = S * n_tiles;
    const int per = (T + XCDS - 1) / XCDS;
    const int r0 = (pid % XCDS) * per;               // this XCD's range [r0, r0 + len)
    const int len = min(per, T - r0);
    int j = pid / XCDS;
    if (pid >= per * XCDS || j >= len) return false;
    // The last kMoeTail positions of the range run their tiles of more than
    // 128 rows first and the smaller ones last (each group in list order), so
    // that the tiles still running when the range runs dry are the short
    // ones: a tile of at most 128 rows takes about 0.7 of a full one, and
    // the ragged end of the last round is otherwise about one average tile
    // long.  Workgroup-uniform branch; the permutation stays inside the
    // window, so every tile still runs exactly once.
    const int w0 = max(0, len - kMoeTail);
    if (j >= w0) {
        const int wn = len - w0;
        for (int t = threadIdx.x; t < wn; t += blockDim.x) {
            int sl, nt, e, seg0, rows;
            moe_list_tile(r0 + w0 + t, S, n_tiles, sl, nt);
            moe_find(p, s_off, sl, e, seg0, rows);
            s_tail[t] = rows > 128;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int nbig = 0;
            for (int t = 0; t < wn; ++t) nbig += s_tail[t];
            const int q = j - w0;
            const int want = q < nbig ? 1 : 0;
            int k = q < nbig ? q : q - nbig, pick = 0;
            for (int t = 0; t < wn; ++t)
                if (s_tail[t] == want && k-- == 0) { pick = t; break; }
            s_tail[kMoeTail] = pick;
        }
        __syncthreads();
        j = w0 + s_tail[kMoeTail];
    }
    moe_list_tile(r0 + j, S, n_tiles, slot, ntile);
    return true;
}

template <int KIND> struct MoePolicy { typedef mfma2::PolicyI8<DmaCfg> type; };   // MOE_S8, MOE_S8_I32
template <> struct MoePolicy<MOE_BF16> { typedef mfma2::PolicyH16<DmaCfg, true> type; };
template <> struct MoePolicy<MOE_F16> { typedef mfma2::PolicyH16<DmaCfg, false> type; };

template <int KIND>
__global__ __launch_bounds__(DmaCfg::NT, 1) void moe_grouped_dma_kernel(MoeArgs p) {
    namespace M2 = mfma2;
    typedef typename MoePolicy<KIND>::type P;
    constexpr int ES = MoeElem<KIND>::SIZE;
    __shared__ __attribute__((aligned(1024))) int8_t stage0[2 * M2::OPER];
    __shared__ __attribute__((aligned(1024))) int8_t stage1[2 * M2::OPER];
    __shared__ int32_t s_rows_tok[M2::BM];
    __shared__ int32_t s_off[kMaxExperts + 1];
    moe_load_offsets(p, s_off);
    int slot, ntile, e, seg0, seg_rows;
    __shared__ int s_tail[kMoeTail + 1];
    if (!moe_dma_coords(p, s_off, blockIdx.x, p.N / M2::BN, slot, ntile, s_tail)) return;   // whole workgroup exits
    if (!moe_find(p, s_off, slot, e, seg0, seg_rows)) return;
    const int n_base = ntile * M2::BN;
    for (int r = threadIdx.x; r < M2::BM; r += DmaCfg::NT)
        s_rows_tok[r] = p.sorted_ids[seg0 + min(r, seg_rows - 1)];
    __syncthreads();
    const int in_div = p.topk_w ? 1 : p.topk;
    const int x_rows = p.topk_w ? p.size_m : (p.size_m + p.topk - 1) / p.topk;
    const int kb = p.K * ES;   // row length in bytes
    M2::DmaRows<true, false> d;
    d.a = M2::make_dma_gathered<DmaCfg>(p.x, (uint32_t)((int64_t)x_rows * kb),
                                        [&](int r) { return (s_rows_tok[r] / in_div) * kb; });
    d.b = M2::make_dma_interior<DmaCfg>(p.w + (int64_t)e * p.N * kb, (uint32_t)((int64_t)p.N * kb),
                                        kb, n_base * kb);
    // A wave whose 128 tile rows are all padding (the expert's last tile
    // holds at most 128 rows) only moves its share of each stage.
    if ((int)((threadIdx.x >> 6) / DmaCfg::WAVES_N) * DmaCfg::WM >= seg_rows) {
        M2::mainloop_dma_only<DmaCfg>(stage0, stage1, d, kb);
        return;
    }
    M2::AccTile<P> acc;
    M2::mainloop<P>(stage0, stage1, d, kb, acc);
    if constexpr (KIND == MOE_S8_I32) {
        // int32 rows staged per wave in two halves of 64 rows and written as
        // 16-byte units of the pair's output row; padding rows are skipped.
        const int wave = threadIdx.x >> 6;
        const int wr = (wave / DmaCfg::WAVES_N) * DmaCfg::WM;
        const int wc = n_base + (wave % DmaCfg::WAVES_N) * DmaCfg::WN;
        int8_t *scratch = (wave < 4 ? stage0 : stage1) + (wave & 3) * (DmaCfg::WM / 2 * 256);
        M2::store_x32x4_staged<P>(
            acc, scratch, [&](int, int, const v4i &v) { return v; },
            [&](int r) -> int32_t * {
                return wr + r < seg_rows ? static_cast<int32_t *>(p.out) + (int64_t)s_rows_tok[wr + r] * p.N + wc
                                         : nullptr;
            });
        return;
    } else if constexpr (KIND != MOE_S8) {
        if ((reinterpret_cast<uintptr_t>(p.out) & 15u) == 0) {
            // Rows staged per wave in LDS and written as 16-byte units of the
            // token's output row; padding rows of a partial tile are skipped.
            const int wave = threadIdx.x >> 6;
            const int wr = (wave / DmaCfg::WAVES_N) * DmaCfg::WM;
            const int wc = n_base + (wave % DmaCfg::WAVES_N) * DmaCfg::WN;
            int8_t *scratch = (wave < 4 ? stage0 : stage1) + (wave & 3) * (DmaCfg::WM * 128);
            M2::store_bf16x4_staged<P>(
                acc, scratch,
                [&](int r, int, const v4f &v) {
                    const float tw = p.topk_w ? p.topk_w[s_rows_tok[wr + r]] : 1.0f;
                    uint16_t h[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float y = p.topk_w ? v[q] * tw : v[q];
                        h[q] = KIND == MOE_BF16 ? f32_to_bf16_rne(y) : f32_to_f16_rne(y);
                    }
                    return v2i{(int)((uint32_t)h[0] | ((uint32_t)h[1] << 16)),
                               (int)((uint32_t)h[2] | ((uint32_t)h[3] << 16))};
                },
                [&](int r) -> uint16_t * {
                    return wr + r < seg_rows ? static_cast<uint16_t *>(p.out) + (int64_t)s_rows_tok[wr + r] * p.N + wc
                                             : nullptr;
                });
            return;
        }
        M2::for_each_quad<P>(acc, [&](int ml, int nl, const v4f &v) {
            moe_store_h<KIND>(p, s_rows_tok, seg_rows, ml, n_base + nl, v);
        });
        return;
    } else {
        // Epilogue: scales (per token row, per expert column) fetched once per
        // lane; the wave tile is staged in LDS and written as full 128-byte rows
        // of the token's output row; padding rows of a partial tile are skipped.
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int wr = (wave / DmaCfg::WAVES_N) * DmaCfg::WM;
        const int wc = n_base + (wave % DmaCfg::WAVES_N) * DmaCfg::WN;
        const float *swe = p.sw + (int64_t)e * p.N;
        float sam[P::TI], post[P::TI];
        v4f swv[P::TJ];
#pragma unroll
        for (int i = 0; i < P::TI; ++i) {
            const int tok = s_rows_tok[wr + i * 16 + (lane & 15)];
            sam[i] = p.sa[tok / in_div];
            post[i] = p.topk_w ? p.topk_w[tok] : 1.0f;
        }
#pragma unroll
        for (int j = 0; j < P::TJ; ++j) swv[j] = *reinterpret_cast<const v4f *>(swe + wc + j * 16 + (lane >> 4) * 4);
        int8_t *scratch = (wave < 4 ? stage0 : stage1) + (wave & 3) * (DmaCfg::WM * DmaCfg::WN * 2);
        auto dst = [&](int r) -> uint16_t * {
            return wr + r < seg_rows ? static_cast<uint16_t *>(p.out) + (int64_t)s_rows_tok[wr + r] * p.N + wc
                                     : nullptr;
        };
        if (p.topk_w) M2::store_w8a8_bf16_staged<P, true>(acc, scratch, sam, post, swv, dst);
        else M2::store_w8a8_bf16_staged<P, false>(acc, scratch, sam, post, swv, dst);
    }
}

// Decode-sized MoE (size_m <= 64): one launch over (N / (16 NB) column
// groups) x E experts x (size_m / 16 RF row blocks), no offsets kernel in
// front.  A workgroup of 16 waves finds its expert's rows from the ids
// (moe_decode_rows) and exits when its block of them is empty; otherwise,
// as the dense last-rows pass (gemm_s8_rcr_rows_staged_kernel; with RF * CH
// < 16 only the first RF * CH waves multiply), it streams its 16 RF gathered A rows
// (pair p's input row, through sorted_token_ids; rows past the expert's
// count point past the input and land as zeros) and its 16 NB rows of the
// expert's weight slab through LDS in K stages of SB bytes, DEPTH in
// flight, 16-byte unit u of stage row r at slot u ^ (r & 15).  Wave w owns
// 64-byte chunk w % CH of every stage (CH = SB / 64) and A fragments
// w / CH + (16 / CH) i against all NB weight fragments (the int8 16x16x64 or
// the 16-bit 16x16x32 MFMA, the same 16 bytes per lane); the chunk partials
// are added in chunk order through LDS and the waves run the tile path's
// per-quad epilogues (moe_store, moe_store_i32, moe_store_h).
template <int KIND, int RF, int NB, int SB, int DEPTH>
__global__ __launch_bounds__(1024) void moe_rows_staged_kernel(MoeArgs p) {
    constexpr int WAVES = 16, CH = SB / 64;
    // fewer (fragment, chunk) pairs than waves: the first RF * CH multiply
    constexpr bool ALL = RF * CH >= WAVES;
    constexpr int FPW = ALL ? RF * CH / WAVES : 1;
    constexpr int FSTEP = WAVES / CH;
    constexpr int ROWS = 16 * RF + 16 * NB;
    constexpr int STAGE = ROWS * SB;
    constexpr int UPR = SB / 16;
    constexpr int NI = ROWS * UPR / 64;
    constexpr int HI = (NI + WAVES - 1) / WAVES, LO = NI / WAVES;
    constexpr bool INT = KIND == MOE_S8 || KIND == MOE_S8_I32;
    constexpr int ES = MoeElem<KIND>::SIZE;
    typedef typename std::conditional<INT, v4i, v4f>::type Acc;
    static_assert((!ALL || RF * CH % WAVES == 0) && UPR >= 16 && (ROWS * UPR) % 64 == 0 && DEPTH >= 2 &&
                      DEPTH <= 4 && DEPTH * STAGE + 64 * RF <= 160 * 1024 && RF * NB * CH * 1024 + 64 * RF <= 160 * 1024,
                  "stage split");
    // dynamic LDS: the stages (then the partial sums), then the A rows' pair ids
    constexpr int MAIN = DEPTH * STAGE > RF * NB * CH * 1024 ? DEPTH * STAGE : RF * NB * CH * 1024;
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];
    int32_t *s_tok = reinterpret_cast<int32_t *>(lds + MAIN);
    const int e = blockIdx.y;
    int o0, rows;
    moe_decode_rows(p, e, o0, rows);
    // blockIdx.z: 16 RF-row block of the expert's rows
    o0 += blockIdx.z * 16 * RF;
    rows = min(rows - (int)blockIdx.z * 16 * RF, 16 * RF);
    if (rows <= 0) return;   // whole workgroup: no rows of this expert in this block
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16 * NB;
    const int kb = p.K * ES;
    const int in_div = p.topk_w ? 1 : p.topk;
    const int x_rows = p.topk_w ? p.size_m : (p.size_m + p.topk - 1) / p.topk;
    for (int r = threadIdx.x; r < 16 * RF; r += blockDim.x) s_tok[r] = r < rows ? p.sorted_ids[o0 + r] : -1;
    __syncthreads();
    const v4i ra = mfma2::make_rsrc(p.x, (uint32_t)((int64_t)x_rows * kb));
    const v4i rb = mfma2::make_rsrc(p.w + (int64_t)e * p.N * kb, (uint32_t)((int64_t)p.N * kb));
    auto dma_stage = [&](int st, int8_t *buf) {
        const int k0 = st * SB;
        for (int j = wave; j < NI; j += WAVES) {
            const int idx = 64 * j + lane;
            const int r = idx / UPR, slot = idx % UPR;
            const int unit = slot ^ (r & 15);
            if (r < 16 * RF) {
                const int tok = s_tok[r];
                const int base = tok >= 0 ? (tok / in_div) * kb : x_rows * kb;   // past the input: zeros
                mfma2::dma16(ra, base + 16 * unit, k0, buf + j * 1024);
            } else {
                mfma2::dma16(rb, (n0 + r - 16 * RF) * kb + 16 * unit, k0, buf + j * 1024);
            }
        }
    };
    const bool hi = NI % WAVES == 0 || wave < NI % WAVES;
    const int ns = kb / SB;
    for (int st = 0; st < DEPTH && st < ns; ++st) dma_stage(st, lds + st * STAGE);
    const int c = wave % CH, f0 = wave / CH;
    const bool active = ALL || wave < RF * CH;   // wave-uniform
    Acc acc[FPW][NB];
#pragma unroll
    for (int i = 0; i < FPW; ++i)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[i][nb] = Acc{0, 0, 0, 0};
    const int sl = 16 * ((4 * c + g) ^ r16);
    for (int st = 0; st < ns; ++st) {
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
        for (int nb = 0; nb < NB; ++nb)
            bv[nb] = *reinterpret_cast<const v4i *>(buf + (16 * RF + 16 * nb + r16) * SB + sl);
#pragma unroll
        for (int i = 0; i < FPW; ++i) {
            const v4i av = *reinterpret_cast<const v4i *>(buf + (16 * (f0 + FSTEP * i) + r16) * SB + sl);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                if constexpr (INT) acc[i][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bv[nb], av, acc[i][nb], 0, 0, 0);
                else acc[i][nb] = mfma16x16x32_h<KIND == MOE_BF16>(bv[nb], av, acc[i][nb]);
            }
        }
        }
        __syncthreads();
        if (st + DEPTH < ns) dma_stage(st + DEPTH, buf);
    }
    Acc *part = reinterpret_cast<Acc *>(lds);
    if (active) {
#pragma unroll
        for (int i = 0; i < FPW; ++i)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) part[(((f0 + FSTEP * i) * NB + nb) * CH + c) * 64 + lane] = acc[i][nb];
    }
    __syncthreads();
    const float *swe = INT && p.sw ? p.sw + (int64_t)e * p.N : nullptr;
    for (int q = wave; q < RF * NB; q += WAVES) {
        const int f = q % RF, nb = q / RF;
        Acc sum = part[((f * NB + nb) * CH) * 64 + lane];
#pragma unroll
        for (int cc = 1; cc < CH; ++cc) {
            const Acc v = part[((f * NB + nb) * CH + cc) * 64 + lane];
            if constexpr (INT)
                sum = v4i{(int)((uint32_t)sum[0] + (uint32_t)v[0]), (int)((uint32_t)sum[1] + (uint32_t)v[1]),
                          (int)((uint32_t)sum[2] + (uint32_t)v[2]), (int)((uint32_t)sum[3] + (uint32_t)v[3])};
            else
                sum = v4f{sum[0] + v[0], sum[1] + v[1], sum[2] + v[2], sum[3] + v[3]};
        }
        const int ml = 16 * f + r16, nn = n0 + 16 * nb + 4 * g;
        if constexpr (KIND == MOE_S8) moe_store(p, s_tok, rows, in_div, swe, ml, nn, sum);
        else if constexpr (KIND == MOE_S8_I32) moe_store_i32(p, s_tok, rows, ml, nn, sum);
        else moe_store_h<KIND>(p, s_tok, rows, ml, nn, sum);
    }
}

// Decode-sized int8 MoE with a few rows per expert (K % 1024 == 0): one
// launch over (N / 4 column groups) x E experts of 4 waves, no MFMA, the
// layout of the dense one-row kernel (gemm_s8_rcr_row1_kernel).  Wave w
// streams row n0 + w of the expert's weight slab, 16 bytes per lane of every
// kilobyte, straight into registers and takes v_dot4_i32_i8 of it against
// the same bytes of up to RMAX of the expert's gathered A rows (L2 hits);
// an expert with more rows takes further passes over the slab rows (L2
// hits).  Wave butterflies and LDS gather the 4 column sums of each row and
// the tile path's per-quad epilogue (moe_store / moe_store_i32) writes them:
// int32 sums are exact, so the output is bit-identical to the MFMA paths.
template <int KIND, int RMAX, int BT>
__global__ __launch_bounds__(256) void moe_row_kernel(MoeArgs p) {
    static_assert(KIND == MOE_S8 || KIND == MOE_S8_I32, "int8 kinds");
    __shared__ int32_t s_tok[RMAX];
    __shared__ int colsum[RMAX][4];
    const int e = blockIdx.y;
    int o0, rows;
    moe_decode_rows(p, e, o0, rows);
    if (rows <= 0) return;   // whole workgroup: no rows routed to this expert
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * 4;
    const int kb = p.K;
    const int nch = kb >> 10;
    const int in_div = p.topk_w ? 1 : p.topk;
    const int8_t *brow = p.w + ((int64_t)e * p.N + n0 + wave) * kb + lane * 16;
    const float *swe = KIND == MOE_S8 ? p.sw + (int64_t)e * p.N : nullptr;
    for (int r0 = 0; r0 < rows; r0 += RMAX) {
        const int nr = min(RMAX, rows - r0);
        if (threadIdx.x < RMAX) s_tok[threadIdx.x] = threadIdx.x < nr ? p.sorted_ids[o0 + r0 + threadIdx.x] : 0;
        __syncthreads();
        const int8_t *arow[RMAX];
#pragma unroll
        for (int r = 0; r < RMAX; ++r)
            arow[r] = p.x + (int64_t)(s_tok[r < nr ? r : 0] / in_div) * kb + lane * 16;
        int acc[RMAX];
#pragma unroll
        for (int r = 0; r < RMAX; ++r) acc[r] = 0;
        for (int c0 = 0; c0 < nch; c0 += BT) {
            v4i bv[BT], av[BT][RMAX];
#pragma unroll
            for (int u = 0; u < BT; ++u)
#pragma unroll
                for (int r = 0; r < RMAX; ++r)
                    av[u][r] = r < nr ? *reinterpret_cast<const v4i *>(arow[r] + (int64_t)(c0 + u) * 1024)
                                      : v4i{0, 0, 0, 0};
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < BT; ++u)
                bv[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(brow + (int64_t)(c0 + u) * 1024));
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < BT; ++u)
#pragma unroll
                for (int r = 0; r < RMAX; ++r)
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[r] = __builtin_amdgcn_sdot4(av[u][r][q], bv[u][q], acc[r], false);
        }
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1)
                acc[r] = (int)((uint32_t)acc[r] + (uint32_t)__shfl_xor(acc[r], off, 64));
            if (lane == 0) colsum[r][wave] = acc[r];
        }
        __syncthreads();
        if (threadIdx.x < nr) {
            const int r = threadIdx.x;
            const v4i v{colsum[r][0], colsum[r][1], colsum[r][2], colsum[r][3]};
            if constexpr (KIND == MOE_S8) moe_store(p, s_tok, nr, in_div, swe, r, n0, v);
            else moe_store_i32(p, s_tok, nr, r, n0, v);
        }
        __syncthreads();   // s_tok and colsum are rewritten by the next pass
    }
}

// Offsets, then the grouped GEMM (DMA path when the problem fits it).
template <int KIND>
int32_t launch_moe(const MoeArgs &p, const int32_t *expert_ids, int32_t *expert_counts,
                   bool out_ok, hipStream_t stream) {
    constexpr int ES = MoeElem<KIND>::SIZE;
    // Upper bound on ragged m-tiles: sum_e ceil(cnt_e / BM) <= ceil(size_m / BM) + E.
    const int slots = (p.size_m + BM - 1) / BM + p.E;
    // The DMA path needs whole 128-byte K stages, N a multiple of 256, 16-byte
    // aligned operands, byte offsets that fit 32 bits (per input / per expert
    // slab) and what its epilogue needs (out_ok).
    const int64_t kb = (int64_t)p.K * ES;
    const int64_t x_rows = p.topk_w ? p.size_m : (p.size_m + p.topk - 1) / p.topk;
    const bool fast = kb % mfma2::BK == 0 && p.N % mfma2::BN == 0 && mfma::aligned16(p.x) &&
                      mfma::aligned16(p.w) && x_rows * kb < (1ll << 31) &&
                      (int64_t)p.N * kb < (1ll << 31) && out_ok;
    // Decode launches (size_m <= 64) find their rows from the ids themselves
    // and write the counts and offsets: no offsets kernel in front (N =
    // 14336, K = 4096, E = 8, top-2, 2 rotated weight sets, graph replay: 1 /
    // 2 / 4 / 8 / 16 tokens 27.3 / 60.4 / 72.6 / 86.2 / 98.2 -> 22.4 / 56.0 /
    // 67.9 / 81.2 / 95.5 us, bit-identical).
    MoeArgs q = p;
    q.expert_ids = expert_ids;
    q.counts = expert_counts;
    if constexpr (KIND == MOE_S8 || KIND == MOE_S8_I32) {
        // 3-6 pairs: the dot4 row kernel, 2 rows per pass over the weights
        // (2 / 3 tokens: 53.4 / 53.4 -> 48.0 / 48.0 us against the staged
        // kernel's 16-row blocks; at 2 pairs 22.5 against 22.4 us, at 8
        // 65.9 against 64.8 us: those stay staged)
        if (fast && p.size_m > 2 && p.size_m <= 6 && kb % 1024 == 0 && p.N % 4 == 0) {
            if (kb % 2048 == 0)
                hipLaunchKernelGGL((moe_row_kernel<KIND, 2, 2>), dim3(p.N / 4, p.E), dim3(256), 0, stream, q);
            else
                hipLaunchKernelGGL((moe_row_kernel<KIND, 2, 1>), dim3(p.N / 4, p.E), dim3(256), 0, stream, q);
            return launch_status();
        }
    }
    if (fast && p.size_m <= 64 && kb % 512 == 0) {
        // decode-sized.  N = 14336, K = 4096, E = 8, top-2: 1 / 4 / 16 tokens
        // (2 / 5 / 7 experts) in 27.4 / 62.3 / 99.0 us (with the offsets
        // kernel) against 43.5 / 100.5 / 117.8 on 256-row tiles; at size_m
        // 96 / 128 8 row fragments ran level with the tiles (123 us), so
        // larger size_m stays on them.
        const int nb = mfma2::last_rows_col_frags(p.N);
        // blocks of 16 rows up to 32 pairs, of 32 above (blockIdx.z): an
        // expert's few rows stage fewer padding rows (N = 14336, K = 4096,
        // 1 / 8 / 16 / 32 tokens top-2: 22.6 / 80.7 / 95.5 / 106.6 -> 21.6 /
        // 77.8 / 92.7 / 100.1 us against one block of 32 or 64 rows)
        const int rfz = p.size_m <= 32 ? 1 : 2;
#define BK_MOEROWS(RF, NB, SB, DEPTH)                                                                        \
        if (rfz == (RF) && nb == (NB)) {                                                                     \
            hipLaunchKernelGGL((moe_rows_staged_kernel<KIND, RF, NB, SB, DEPTH>),                            \
                               dim3(p.N / (16 * (NB)), p.E, (p.size_m + 16 * (RF) - 1) / (16 * (RF))),      \
                               dim3(1024),                                                                   \
                               std::max((size_t)(DEPTH) * (16 * (RF) + 16 * (NB)) * (SB),                    \
                                        (size_t)(RF) * (NB) * ((SB) / 64) * 1024) + 64 * (RF),               \
                               stream, q);                                                                   \
            return launch_status();                                                                          \
        }
        BK_MOEROWS(1, 1, 512, 3)
        BK_MOEROWS(1, 2, 512, 3)
        BK_MOEROWS(1, 4, 512, 3)
        BK_MOEROWS(2, 1, 512, 3)
        BK_MOEROWS(2, 2, 512, 3)
        BK_MOEROWS(2, 4, 512, 3)
#undef BK_MOEROWS
    }
    hipLaunchKernelGGL(moe_offsets_kernel, dim3(1), dim3(1024), 0, stream, expert_ids, p.size_m, p.E,
                       expert_counts, const_cast<int32_t *>(p.offsets));
    if (hipPeekAtLastError() != hipSuccess) return kLaunch;
    if (fast) {
        const int work = slots * (p.N / mfma2::BN);
        const int padded = (work + 7) / 8 * 8;   // whole XCD groups
        hipLaunchKernelGGL((moe_grouped_dma_kernel<KIND>), dim3(padded), dim3(DmaCfg::NT), 0, stream, p);
    } else {
        dim3 grid(slots, (p.N + BN - 1) / BN);
        hipLaunchKernelGGL((moe_grouped_kernel<KIND>), grid, dim3(NT), 0, stream, p);
    }
    return launch_status();
}

}  // namespace
}  // namespace bk

using namespace bk;

extern "C" {

int32_t baracuda_kernels_moe_s8_grouped_bf16_gfx950_can_implement(
    int32_t num_experts, int32_t topk, int32_t size_m, int32_t size_n, int32_t size_k) {
    if (num_experts <= 0 || topk <= 0) return kInvalid;
    if (size_m <= 0 || size_n <= 0 || size_k <= 0) return kInvalid;
    if (topk > num_experts) return kInvalid;
    if (num_experts > kMaxExperts) return kUnsupported;
    return kOk;
}

size_t baracuda_kernels_moe_s8_grouped_bf16_gfx950_workspace_size(
    int32_t num_experts, int32_t topk, int32_t size_m, int32_t size_n, int32_t size_k) {
    (void)num_experts; (void)topk; (void)size_m; (void)size_n; (void)size_k;
    return 0;
}

// Argument order follows baracuda_kernels_moe_wmma_bf16_run (moe_wmma.cu:154-175)
// with the two W8A8 scale vectors inserted before the workspace.
int32_t baracuda_kernels_moe_s8_grouped_bf16_gfx950_run(
    const void *input, const void *weights, const int32_t *sorted_token_ids,
    const int32_t *expert_ids, const float *topk_weights, void *output,
    int32_t *expert_counts, int32_t *expert_offsets, int32_t num_experts, int32_t topk,
    int32_t size_m, int32_t size_n, int32_t size_k, const float *scale_a, const float *scale_w,
    void *workspace, size_t workspace_bytes, void *stream_ptr) {
    (void)workspace; (void)workspace_bytes;
    if (!input || !weights || !sorted_token_ids || !expert_ids || !output || !expert_counts ||
        !expert_offsets || !scale_a || !scale_w)
        return kInvalid;
    int32_t st = baracuda_kernels_moe_s8_grouped_bf16_gfx950_can_implement(num_experts, topk, size_m,
                                                                           size_n, size_k);
    if (st != kOk) return st;
    MoeArgs p{(const int8_t *)input, (const int8_t *)weights, sorted_token_ids, expert_offsets,
              topk_weights, scale_a, scale_w, output, num_experts, topk, size_m,
              size_n, size_k};
    // The staged W8A8 epilogue writes 16-byte units of output rows and reads
    // 16-byte groups of column scales.
    return launch_moe<MOE_S8>(p, expert_ids, expert_counts,
                              mfma::aligned16(output) && mfma::aligned16(scale_w),
                              (hipStream_t)stream_ptr);
}

// int32-accumulator SKU of the grouped int8 MoE (no counterpart in the
// reference, which has no int8 MoE): the W8A8 SKU's arguments without the
// scales and topk_weights; input row of pair p = sorted_token_ids[p] / topk,
// out[sorted_token_ids[p], n] = acc (int32).  It exposes, for a whole-output
// exact check, the accumulator that the bf16 SKU's epilogue dequantizes.
int32_t baracuda_kernels_moe_s8_grouped_i32_gfx950_can_implement(
    int32_t num_experts, int32_t topk, int32_t size_m, int32_t size_n, int32_t size_k) {
    return baracuda_kernels_moe_s8_grouped_bf16_gfx950_can_implement(num_experts, topk, size_m, size_n, size_k);
}

int32_t baracuda_kernels_moe_s8_grouped_i32_gfx950_run(
    const void *input, const void *weights, const int32_t *sorted_token_ids, const int32_t *expert_ids,
    void *output, int32_t *expert_counts, int32_t *expert_offsets, int32_t num_experts, int32_t topk,
    int32_t size_m, int32_t size_n, int32_t size_k, void *stream_ptr) {
    if (!input || !weights || !sorted_token_ids || !expert_ids || !output || !expert_counts || !expert_offsets)
        return kInvalid;
    int32_t st = baracuda_kernels_moe_s8_grouped_bf16_gfx950_can_implement(num_experts, topk, size_m,
                                                                           size_n, size_k);
    if (st != kOk) return st;
    MoeArgs p{(const int8_t *)input, (const int8_t *)weights, sorted_token_ids, expert_offsets,
              nullptr, nullptr, nullptr, output, num_experts, topk, size_m, size_n, size_k};
    return launch_moe<MOE_S8_I32>(p, expert_ids, expert_counts, mfma::aligned16(output),
                                  (hipStream_t)stream_ptr);
}

// Same ABI as baracuda_kernels_moe_wmma_{f16,bf16}_{run,can_implement}
// (crates/baracuda-kernels-sys/kernels/moe/moe_wmma.cu:121-209): bf16 / f16
// input [*, K] and weights [E, N, K], f32 accumulation, out[row, n] in the
// input type; is_prefill (a tile-shape hint there) has no effect here.
#define BK_MOE_WMMA(TAG, KIND)                                                                     \
    int32_t baracuda_kernels_moe_wmma_##TAG##_can_implement(int32_t num_experts, int32_t topk,    \
                                                            int32_t size_m, int32_t size_n,       \
                                                            int32_t size_k, int32_t is_prefill) { \
        (void)is_prefill;                                                                          \
        return baracuda_kernels_moe_s8_grouped_bf16_gfx950_can_implement(num_experts, topk, size_m,\
                                                                         size_n, size_k);         \
    }                                                                                              \
    int32_t baracuda_kernels_moe_wmma_##TAG##_run(                                                 \
        const void *input, const void *weights, const int32_t *sorted_token_ids,                   \
        const int32_t *expert_ids, const float *topk_weights, void *output,                        \
        int32_t *expert_counts, int32_t *expert_offsets, int32_t num_experts, int32_t topk,        \
        int32_t size_m, int32_t size_n, int32_t size_k, int32_t is_prefill, void *workspace,       \
        size_t workspace_bytes, void *stream_ptr) {                                                \
        (void)is_prefill; (void)workspace; (void)workspace_bytes;                                  \
        if (!input || !weights || !sorted_token_ids || !expert_ids || !output || !expert_counts ||  \
            !expert_offsets)                                                                       \
            return kInvalid;                                                                       \
        int32_t st = baracuda_kernels_moe_s8_grouped_bf16_gfx950_can_implement(                   \
            num_experts, topk, size_m, size_n, size_k);                                            \
        if (st != kOk) return st;                                                                  \
        MoeArgs p{(const int8_t *)input, (const int8_t *)weights, sorted_token_ids, expert_offsets, \
                  topk_weights, nullptr, nullptr, output, num_experts, topk, size_m,               \
                  size_n, size_k};                                                                 \
        return launch_moe<KIND>(p, expert_ids, expert_counts, true, (hipStream_t)stream_ptr);      \
    }

BK_MOE_WMMA(bf16, MOE_BF16)
BK_MOE_WMMA(f16, MOE_F16)
#undef BK_MOE_WMMA

}  // extern "C"
