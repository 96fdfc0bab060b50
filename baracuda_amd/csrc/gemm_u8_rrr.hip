// gemm_u8_rrr.hip -- u8 x u8 RRR GEMM (B row-major [K, N]) and its bias /
// activation family for gfx950: D = sat_u8(rne(act(alpha*acc + beta*C
// [+ bias[n]]))), acc the exact int32 sum of u8 products.
//
// gfx950's int8 MFMA is signed, so operands run through it as u - 128 and the
// kernels add the row / column-sum correction back (gemm_s8_kernels.hpp).
#include <mutex>

#include "gemm_s8_kernels.hpp"

using namespace bk;

// ---- scratch of the allocation-free entry point ------------------------------
// The u8 RRR pre-pass workspace (flipped operands + their sums) of
// baracuda_kernels_gemm_u8_rrr_gfx950_noalloc_run, in a device array of fixed
// size that each GPU the library runs on holds until the process ends.  Host
// code never uses the array's name as an address: the device address comes
// from hipGetSymbolAddress, once per device, with that device current.
static constexpr size_t kU8NoAllocScratchBytes = BARACUDA_U8_RRR_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) int8_t scratch[kU8NoAllocScratchBytes];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device (looked up on first use).
static int32_t current_device_scratch(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return kLaunch;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
            (void)hipGetLastError();   // leave no sticky error for the next call
            return kLaunch;
        }
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return kOk;
}

extern "C" {

// Same ABI as baracuda_kernels_gemm_u8_rrr_sm80_* and its bias family
// (crates/baracuda-kernels-sys/kernels/gemm/gemm_u8_rrr_sm80.cu,
//  gemm_u8_rrr_sm80_bias.cu; bound in crates/baracuda-kernels-sys/src/lib.rs:120-160,462-).
static int32_t check_u8_rrr(int32_t m, int32_t n, int32_t k, int64_t lda, int64_t ldb,
                            const void *c, int64_t ldc, int64_t ldd) {
    if (m <= 0 || n <= 0 || k <= 0) return kInvalid;
    if (lda < k || ldb < n || ldd < n) return kInvalid;
    if (c != nullptr && ldc < n) return kInvalid;
    return kOk;
}

int32_t baracuda_kernels_gemm_u8_rrr_gfx950_can_implement(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd) {
    (void)a; (void)b; (void)d;
    return check_u8_rrr(m, n, k, lda, ldb, c, ldc, ldd);
}

// Optional workspace (256-byte aligned): the operands flipped to u - 128 and
// their (M + N) int32 sums.  Given it, whole-tile problems run a pre-pass and
// then the plain s8 RRR loop; without it the flip and the sums are folded
// into the GEMM loop (slower: the extra registers spill).
size_t baracuda_kernels_gemm_u8_rrr_gfx950_workspace_size(int32_t m, int32_t n, int32_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || m % 256 || n % 256 || k % 128) return 0;
    return u8_rrr_workspace_bytes(m, n, k);
}

int32_t baracuda_kernels_gemm_u8_rrr_gfx950_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta,
    void *workspace, size_t workspace_bytes, void *stream) {
    int32_t st = check_u8_rrr(m, n, k, lda, ldb, c, ldc, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d) return kInvalid;
    S8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, (const int8_t *)c, ldc, d, ldd,
             alpha, beta, nullptr, nullptr, nullptr};
    return launch_u8_rrr<ACT_NONE, float>(p, (hipStream_t)stream, workspace, workspace_bytes);
}

// The same GEMM with no workspace argument and no allocation: whole-tile
// problems run the pre-pass into this device's `scratch` (they are rejected
// with kWorkspace when the pre-pass needs more than its size); other shapes
// run the in-loop path, which needs no scratch.  The pre-pass rewrites every
// byte of scratch it reads (the column sums are zeroed by its first kernel),
// so nothing carries over from the previous call.
int32_t baracuda_kernels_gemm_u8_rrr_gfx950_noalloc_run(
    int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,
    const void *c, int64_t ldc, void *d, int64_t ldd, float alpha, float beta, void *stream) {
    int32_t st = check_u8_rrr(m, n, k, lda, ldb, c, ldc, ldd);
    if (st != kOk) return st;
    if (!a || !b || !d) return kInvalid;
    S8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, (const int8_t *)c, ldc, d, ldd,
             alpha, beta, nullptr, nullptr, nullptr};
    if (!u8_rrr_prepass_eligible(p)) return launch_u8_rrr<ACT_NONE, float>(p, (hipStream_t)stream);
    if (u8_rrr_workspace_bytes(m, n, k) > kU8NoAllocScratchBytes) return kWorkspace;
    void *ws = nullptr;
    st = current_device_scratch(&ws);
    if (st != kOk) return st;
    return launch_u8_rrr<ACT_NONE, float>(p, (hipStream_t)stream, ws, kU8NoAllocScratchBytes);
}

#define BK_U8_RRR_BIAS(EPISFX, ACTV, BSFX, BTY)                                                      \
    int32_t baracuda_kernels_gemm_u8_rrr_gfx950_##EPISFX##_##BSFX##_can_implement(                  \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,     \
        const void *c, int64_t ldc, const void *d, int64_t ldd) {                                    \
        (void)a; (void)b; (void)d;                                                                   \
        return check_u8_rrr(m, n, k, lda, ldb, c, ldc, ldd);                                         \
    }                                                                                                \
    int32_t baracuda_kernels_gemm_u8_rrr_gfx950_##EPISFX##_##BSFX##_run(                            \
        int32_t m, int32_t n, int32_t k, const void *a, int64_t lda, const void *b, int64_t ldb,     \
        const void *c, int64_t ldc, void *d, int64_t ldd, const void *bias, float alpha, float beta, \
        void *workspace, size_t workspace_bytes, void *stream) {                                     \
        int32_t st = check_u8_rrr(m, n, k, lda, ldb, c, ldc, ldd);                                   \
        if (st != kOk) return st;                                                                    \
        if (!a || !b || !d || !bias) return kInvalid;                                                \
        S8Args p{m, n, k, (const int8_t *)a, lda, (const int8_t *)b, ldb, (const int8_t *)c, ldc, d, \
                 ldd, alpha, beta, nullptr, nullptr, bias};                                          \
        return launch_u8_rrr<ACTV, BTY>(p, (hipStream_t)stream, workspace, workspace_bytes);         \
    }

BK_U8_RRR_BIAS(bias, ACT_BIAS, f32, float)
BK_U8_RRR_BIAS(bias_relu, ACT_BIAS_RELU, f32, float)
BK_U8_RRR_BIAS(bias_gelu, ACT_BIAS_GELU, f32, float)
BK_U8_RRR_BIAS(bias_silu, ACT_BIAS_SILU, f32, float)
BK_U8_RRR_BIAS(bias, ACT_BIAS, i32, int32_t)
BK_U8_RRR_BIAS(bias_relu, ACT_BIAS_RELU, i32, int32_t)
BK_U8_RRR_BIAS(bias_gelu, ACT_BIAS_GELU, i32, int32_t)
BK_U8_RRR_BIAS(bias_silu, ACT_BIAS_SILU, i32, int32_t)
#undef BK_U8_RRR_BIAS

}  // extern "C"
