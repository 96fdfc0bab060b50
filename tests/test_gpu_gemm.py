"""GPU parity of the int8 / FP8 RCR GEMMs against the CPU oracle.

Bars: int32 accumulators and int8 outputs bit-exact; W8A8 bf16 bit-exact
(same f32 epilogue order as the oracle); FP8 f32 accumulator within 1e-3
relative to the exact f64 sum, with an absolute floor of FP8_FLOOR * sum|a*b| for
sums that cancel; FP8 bf16 within 1 bf16 ulp of the exact value (same floor).
The floor is the gfx950 f8f6f4 MFMA's own internal summation error: hipBLASLt
(torch._scaled_mm) on the same inputs shows the same error (max 4.6e-5 *
sum|a*b| at K=32, 4.2e-6 at K=1024), which test_fp8_matches_hipblaslt checks.
"""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from oracle import oracle as O
from oracle.inputs import int8_uniform, rng, w8a8
from tests.gpu_util import FP8_FLOOR, FP8_FLOOR_CONFIG3, bf16_ulp, dev, host_bits16, sync

pytestmark = pytest.mark.gpu

GOLD = __import__("pathlib").Path(__file__).resolve().parent / "golden"
REF_SHAPES = [(64, 64, 32), (128, 128, 128), (256, 128, 64), (100, 70, 50)]   # int8_rrr_smoke.rs / fp8 smokes


def _i32(a, b):
    m, k = a.shape
    n = b.shape[0]
    d = torch.full((m, n), -7, dtype=torch.int32, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.I32)).run(dev(a), dev(b), d)
    sync()
    return d.cpu().numpy()


def test_config1_256_cubed_matches_golden_and_oracle(gpu):
    z = np.load(GOLD / "config1_s8_rcr_256.npz")
    print("case: config1 i32 256^3", flush=True)
    got = _i32(z["a"], z["b"])
    assert np.array_equal(got, z["c"])
    assert np.array_equal(got, O.contraction_s8_i32(z["a"], z["b"].T))


@pytest.mark.parametrize("shape", REF_SHAPES + [(1, 1, 1), (3, 300, 17), (257, 513, 129), (512, 256, 4096)])
def test_i32_ragged_shapes(gpu, shape):
    m, n, k = shape
    print(f"case: i32 {shape}", flush=True)
    g = rng(m * 7 + n * 3 + k)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    assert np.array_equal(_i32(a, b), O.gemm_s8_rcr_i32(a, b, nthreads=8))


# Shapes on the LDS-DMA path (whole 256x256 tiles, K % 128 == 0): one stage,
# an even and an odd number of stages, several tiles per XCD group.
DMA_SHAPES = [(256, 256, 128), (256, 512, 256), (512, 256, 384), (768, 1024, 640), (2048, 512, 1152)]


@pytest.mark.parametrize("shape", DMA_SHAPES)
def test_i32_dma_path_shapes(gpu, shape):
    m, n, k = shape
    print(f"case: i32 dma {shape}", flush=True)
    g = rng(m + 3 * n + 7 * k)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    assert np.array_equal(_i32(a, b), O.gemm_s8_rcr_i32(a, b, nthreads=8))


@pytest.mark.parametrize("shape", DMA_SHAPES[:3])
def test_w8a8_dma_path_shapes(gpu, shape):
    a, w, sa, sw = w8a8(*shape, seed=13)
    assert np.array_equal(_w8a8(a, w, sa, sw), O.gemm_w8a8_bf16(a, w, sa, sw, nthreads=8))


# Edge tiles on the LDS-DMA path (K % 128 == 0, M or N not a multiple of
# 256): operand rows past M / N load as zeros, stores past them are masked.
# N % 8 == 4 and N % 4 != 0 take the per-quad epilogue inside the same kernel.
EDGE_SHAPES = [(300, 520, 384), (1, 256, 4096), (257, 264, 128), (100, 68, 256), (70, 70, 128),
               (513, 300, 1152), (4000, 512, 256)]


@pytest.mark.parametrize("shape", EDGE_SHAPES)
def test_edge_tiles_dma_path(gpu, shape):
    m, n, k = shape
    print(f"case: edge dma {shape}", flush=True)
    g = rng(m + 5 * n + 11 * k)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    assert np.array_equal(_i32(a, b), O.gemm_s8_rcr_i32(a, b, nthreads=8))
    c = int8_uniform(g, (m, n))
    d = torch.full((m, n), 99, dtype=torch.int8, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k)).run(dev(a), dev(b), d, c=dev(c), alpha=0.002, beta=0.75)
    sync()
    assert np.array_equal(d.cpu().numpy(), O.gemm_s8_rcr_s8(a, b, 0.002, 0.75, c))
    a8, w8, sa, sw = w8a8(m, n, k, seed=m + n)
    assert np.array_equal(_w8a8(a8, w8, sa, sw), O.gemm_w8a8_bf16(a8, w8, sa, sw, nthreads=8))


def test_w8a8_m4000_and_m4097_sampled_rows(gpu):
    # Off-grid token counts at the config-2 width: the last tile row is partial
    # (160 of 256 rows at M = 4000, 1 row at M = 4097); rows on both sides of
    # every tile-row boundary and the edge rows are compared bit-exact, plus
    # the exact int32 column-sum identity over the whole output.
    for m in (4000, 4097):
        print(f"case: w8a8 M={m} N=K=4096", flush=True)
        a, w, sa, sw = w8a8(m, 4096, 4096, seed=m)
        got = _w8a8(a, w, sa, sw)
        rows = [0, 255, 256, 3839, 3840, 3841, m - 2, m - 1] + list(rng(m).integers(0, m, 8))
        for r in rows:
            want = O.gemm_w8a8_bf16(a, w, sa, sw, rows=(int(r), int(r) + 1), nthreads=8)
            assert np.array_equal(got[r], want[0]), (m, r)
        d = torch.empty((m, 4096), dtype=torch.int32, device="cuda:0")
        P.IntGemmPlan.select(P.IntGemmDescriptor(m, 4096, 4096, output=P.ElementKind.I32)).run(dev(a), dev(w), d)
        sync()
        colsum = d.to(torch.int64).sum(0).cpu().numpy()
        assert np.array_equal(colsum, w.astype(np.int64) @ a.astype(np.int64).sum(0))


def _ws(plan):
    n = plan.workspace_size()
    return torch.full((max(n, 1),), 0x5A, dtype=torch.uint8, device="cuda:0") if n else None


def test_tail_split_w8a8_m4296_bit_identical(gpu):
    # M = 4296 at the config-2 width: 272 tiles, the 17th tile row (200 valid
    # rows) runs split along K through the optional workspace; the output
    # equals the unsplit launch's and the oracle's.
    m, n, k = 4296, 4096, 4096
    print("case: tail split w8a8 M=4296", flush=True)
    a, w, sa, sw = w8a8(m, n, k, seed=41)
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16))
    ws = _ws(plan)
    assert ws is not None and plan.workspace_size() == 16 * 16 * 65536 * 4
    outs = []
    for work in (None, ws):
        d = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
        plan.run(dev(a), dev(w), d, scale_a=dev(sa), scale_b=dev(sw), workspace=work)
        sync()
        outs.append(host_bits16(d))
    assert np.array_equal(outs[0], outs[1])
    for r in (0, 4095, 4096, 4295):
        assert np.array_equal(outs[1][r], O.gemm_w8a8_bf16(a, w, sa, sw, rows=(r, r + 1), nthreads=8)[0]), r


@pytest.mark.parametrize("shape", [(300, 1000, 512), (256, 4096, 4096), (129, 520, 1152), (1100, 3000, 256),
                                   (2100, 4100, 256), (300, 512, 1024), (129, 4096, 1024), (512, 2048, 512),
                                   (200, 8192, 512)])
def test_small_tiles_all_epilogues(gpu, shape):
    # Grids of at most 128 256x256 tiles run 128x128 tiles (no workspace)
    # unless row blocks of the last-rows kernel fit one round (K % 512,
    # N % 16): 64-row blocks at 256 x 4096, 300 x 512, 129 x 4096, 512 x 2048,
    # 128-row blocks at 200 x 8192, partial last blocks included; 2100 x 4100
    # (153 tiles) 256x256 edge tiles: int32 exact over the whole
    # output (edge rows / columns included), s8 with C and beta through the
    # staged byte store, W8A8 bf16 on rows at the tile-row boundaries.
    m, n, k = shape
    print(f"case: small tiles {shape}", flush=True)
    g = rng(m + n + 7 * k)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    pi = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.I32))
    d = torch.full((m, n), -7, dtype=torch.int32, device="cuda:0")
    pi.run(dev(a), dev(b), d)
    sync()
    assert np.array_equal(d.cpu().numpy(), O.gemm_s8_rcr_i32(a, b, nthreads=8))
    c = int8_uniform(g, (m, n))
    d8 = torch.full((m, n), 99, dtype=torch.int8, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k)).run(dev(a), dev(b), d8, c=dev(c), alpha=0.002, beta=0.75)
    sync()
    assert np.array_equal(d8.cpu().numpy(), O.gemm_s8_rcr_s8(a, b, 0.002, 0.75, c))
    sa = g.uniform(0.005, 0.02, m).astype(np.float32)
    sw = g.uniform(0.001, 0.01, n).astype(np.float32)
    db = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16)).run(
        dev(a), dev(b), db, scale_a=dev(sa), scale_b=dev(sw))
    sync()
    got = host_bits16(db)
    for r in (0, 127, 128, m - 1):
        assert np.array_equal(got[r], O.gemm_w8a8_bf16(a, b, sa, sw, rows=(r, r + 1), nthreads=8)[0]), r


@pytest.mark.parametrize("shape", [(512, 512, 8192), (300, 520, 4096), (200, 256, 4096), (1024, 768, 4096)])
def test_tail_split_small_grids(gpu, shape):
    # Grids of at most 128 tiles with K >= 4096 on fewer than 64 128x128
    # tiles split every tile along K when given the workspace: int32
    # accumulators exact, s8 with C / beta and a bias epilogue equal the oracle.
    m, n, k = shape
    print(f"case: tail split {shape}", flush=True)
    g = rng(m + 3 * n + k)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    pi = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.I32))
    assert pi.workspace_size() > 0
    d = torch.full((m, n), -7, dtype=torch.int32, device="cuda:0")
    pi.run(dev(a), dev(b), d, workspace=_ws(pi))
    sync()
    assert np.array_equal(d.cpu().numpy(), O.gemm_s8_rcr_i32(a, b, nthreads=8))
    c = int8_uniform(g, (m, n))
    ps = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k))
    d8 = torch.full((m, n), 99, dtype=torch.int8, device="cuda:0")
    ps.run(dev(a), dev(b), d8, c=dev(c), alpha=0.002, beta=0.75, workspace=_ws(ps))
    sync()
    assert np.array_equal(d8.cpu().numpy(), O.gemm_s8_rcr_s8(a, b, 0.002, 0.75, c))
    bias = (g.standard_normal(n) * 8).astype(np.float32)
    pb = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, epilogue=P.EpilogueKind.BiasRelu,
                                                  bias_element=P.ElementKind.F32))
    db = torch.full((m, n), 99, dtype=torch.int8, device="cuda:0")
    pb.run(dev(a), dev(b), db, c=dev(c), alpha=1.0 / 256, beta=0.75, bias=dev(bias), workspace=_ws(pb))
    sync()
    assert np.array_equal(db.cpu().numpy(), O.gemm_s8_epi(a, b, "rcr", 1.0 / 256, 0.75, c, bias, "relu"))


@pytest.mark.parametrize("pad", [8, 4])
def test_w8a8_dma_path_strided_output(gpu, pad):
    # ldd = N + pad: pad 8 keeps the LDS-staged 16-byte stores, pad 4 takes
    # the per-quad epilogue; padding columns must stay untouched.
    m, n, k = 512, 256, 256
    a, w, sa, sw = w8a8(m, n, k, seed=14)
    d = torch.full((m, n + pad), 3.0, dtype=torch.bfloat16, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16)).run(
        dev(a), dev(w), d[:, :n], scale_a=dev(sa), scale_b=dev(sw))
    sync()
    got = host_bits16(d)
    assert np.array_equal(got[:, :n], O.gemm_w8a8_bf16(a, w, sa, sw, nthreads=8))
    assert np.all(d[:, n:].float().cpu().numpy() == 3.0)


def test_i32_extreme_values_no_overflow(gpu):
    # |acc| = 127*127*K stays < 2^31 for K < 133143: all -127 (and -128) inputs.
    m = n = 256
    k = 8192
    a = np.full((m, k), -128, np.int8)
    b = np.full((n, k), -127, np.int8)
    got = _i32(a, b)
    assert np.all(got == 128 * 127 * k)


@pytest.mark.parametrize("pads", [(128, 64), (16, 16), (0, 4096)])
def test_w8a8_dma_path_strided_operands(gpu, pads):
    # Whole 256x256 tiles with lda = K + pad_a, ldb = K + pad_b (16-byte
    # multiples): the LDS-DMA path with row pitches other than K.
    m, n, k = 512, 512, 384
    pa, pb = pads
    print(f"case: w8a8 dma strided lda={k + pa} ldb={k + pb}", flush=True)
    g = rng(31 + pa + pb)
    af = int8_uniform(g, (m, k + pa))
    bf = int8_uniform(g, (n, k + pb))
    sa = g.uniform(0.005, 0.02, m).astype(np.float32)
    sw = g.uniform(0.001, 0.01, n).astype(np.float32)
    d = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16)).run(
        dev(af)[:, :k], dev(bf)[:, :k], d, scale_a=dev(sa), scale_b=dev(sw))
    sync()
    want = O.gemm_w8a8_bf16(np.ascontiguousarray(af[:, :k]), np.ascontiguousarray(bf[:, :k]), sa, sw, nthreads=8)
    assert np.array_equal(host_bits16(d), want)


def test_fp8_dma_path_strided_operands_match_contiguous(gpu):
    # The same operands once contiguous and once with lda = K + 128, ldb =
    # K + 256: the LDS-DMA kernel runs the same MFMA sequence, so the bf16
    # outputs are bit-identical.
    m, n, k = 512, 768, 512
    g = rng(41)
    af = torch.from_numpy(O.f32_to_fp8(g.standard_normal((m, k + 128)).astype(np.float32), "e4m3")).to("cuda:0")
    bf = torch.from_numpy(O.f32_to_fp8(g.standard_normal((n, k + 256)).astype(np.float32), "e4m3")).to("cuda:0")
    plan = P.Fp8GemmPlan.select(P.Fp8GemmDescriptor(m, n, k, output=P.ElementKind.Bf16))
    d1 = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
    d2 = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
    plan.run(af[:, :k], bf[:, :k], d1, scale_a=0.5, scale_b=0.25)
    plan.run(af[:, :k].contiguous(), bf[:, :k].contiguous(), d2, scale_a=0.5, scale_b=0.25)
    sync()
    assert torch.equal(d1.view(torch.int16), d2.view(torch.int16))


def test_i32_strided_leading_dims(gpu):
    g = rng(9)
    m, n, k, lda, ldb, ldd = 200, 136, 96, 112, 128, 160
    a = int8_uniform(g, (m, lda))
    b = int8_uniform(g, (n, ldb))
    d = torch.zeros((m, ldd), dtype=torch.int32, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.I32)).run(
        dev(a)[:, :k], dev(b)[:, :k], d[:, :n])
    sync()
    out = d.cpu().numpy()
    assert np.array_equal(out[:, :n], O.gemm_s8_rcr_i32(a[:, :k], b[:, :k]))
    assert np.all(out[:, n:] == 0)   # untouched padding


@pytest.mark.parametrize("shape", REF_SHAPES)
def test_s8_sat_epilogue_reference_pattern(gpu, shape):
    # int8_smoke.rs:159-172 patterns, alpha = 0.125; 0 mismatches (the reference allows +-1).
    m, n, k = shape
    print(f"case: s8 sat {shape}", flush=True)
    a = ((np.arange(m * k) * 7) % 15 - 7).astype(np.int8).reshape(m, k)
    b = ((np.arange(k * n) * 11) % 13 - 6).astype(np.int8).reshape(n, k)
    d = torch.zeros((m, n), dtype=torch.int8, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k)).run(dev(a), dev(b), d, alpha=0.125)
    sync()
    assert np.array_equal(d.cpu().numpy(), O.gemm_s8_rcr_s8(a, b, 0.125))


def test_s8_sat_with_beta_c(gpu):
    g = rng(12)
    m, n, k = 300, 260, 384
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    c = int8_uniform(g, (m, n))
    d = torch.zeros((m, n), dtype=torch.int8, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k)).run(dev(a), dev(b), d, c=dev(c), alpha=0.002, beta=0.75)
    sync()
    assert np.array_equal(d.cpu().numpy(), O.gemm_s8_rcr_s8(a, b, 0.002, 0.75, c))


def _w8a8(a, w, sa, sw):
    m, k = a.shape
    n = w.shape[0]
    d = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16)).run(
        dev(a), dev(w), d, scale_a=dev(sa), scale_b=dev(sw))
    sync()
    return host_bits16(d)


@pytest.mark.parametrize("shape", [(512, 512, 512), (100, 70, 50), (384, 1024, 256)])
def test_w8a8_bf16_bit_exact(gpu, shape):
    print(f"case: w8a8 {shape}", flush=True)
    a, w, sa, sw = w8a8(*shape, seed=2)
    assert np.array_equal(_w8a8(a, w, sa, sw), O.gemm_w8a8_bf16(a, w, sa, sw, nthreads=8))


def test_w8a8_config2_full_size_sampled_rows(gpu):
    # 4096^3; every row sampled below is compared bit-exact,
    # plus size-independent checks on the whole output.
    print("case: w8a8 4096^3", flush=True)
    a, w, sa, sw = w8a8(4096, 4096, 4096, seed=2)
    got = _w8a8(a, w, sa, sw)
    rows = [0, 1, 255, 256, 1023, 2048, 3071, 4095] + list(rng(21).integers(0, 4096, 24))
    for r in rows:
        want = O.gemm_w8a8_bf16(a, w, sa, sw, rows=(int(r), int(r) + 1), nthreads=8)
        assert np.array_equal(got[r], want[0]), r
    # column-sum identity on the int32 accumulator: sum_m acc[m, n] = (sum_m a[m,:]) . w[n,:]
    d = torch.empty((4096, 4096), dtype=torch.int32, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(4096, 4096, 4096, output=P.ElementKind.I32)).run(dev(a), dev(w), d)
    sync()
    colsum = d.to(torch.int64).sum(0).cpu().numpy()
    assert np.array_equal(colsum, w.astype(np.int64) @ a.astype(np.int64).sum(0))
    rowsum = d.to(torch.int64).sum(1).cpu().numpy()
    assert np.array_equal(rowsum, a.astype(np.int64) @ w.astype(np.int64).sum(0))


@pytest.mark.parametrize("shape", [(130, 70, 200), (256, 256, 256), (300, 520, 384), (512, 768, 1024)])
def test_quantized_linear_w8a8_f32(gpu, shape):
    # general path (K = 200) and the LDS-DMA path with staged 256-byte row
    # stores (whole and edge tiles)
    m, n, k = shape
    a, w, sa, sw = w8a8(m, n, k, seed=8)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    from baracuda_amd.ffi import lib
    tw, ta, tsa, tsw = dev(w), dev(a), dev(sa), dev(sw)   # keep the buffers alive across the call
    st = lib().quantized_linear_w8a8_f32_gfx950_run(m, n, k, tw.data_ptr(), ta.data_ptr(),
                                                    tsa.data_ptr(), tsw.data_ptr(), out.data_ptr(),
                                                    None, 0, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    sync()
    acc = O.gemm_s8_rcr_i32(a, w).astype(np.float32)
    want = (sa[:, None] * sw[None, :]).astype(np.float32) * acc
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("shape", [(130, 70, 200), (256, 256, 256), (300, 520, 384), (512, 768, 1024)])
def test_quantized_linear_w8a8_f64(gpu, shape):
    # compose.cu:27-28 f64 SKU: f64 scales narrowed to f32, y = sa*sw*acc in
    # f32, widened to f64.  The f64 scales carry bits below f32 precision so
    # a kernel that multiplied in f64 would differ.  General path (K = 200),
    # LDS-DMA path with the staged 512-byte row stores (whole and edge tiles).
    m, n, k = shape
    a, w, _, _ = w8a8(m, n, k, seed=18)
    g = rng(19)
    sa = g.uniform(0.005, 0.02, m)            # f64, not f32-representable
    sw = g.uniform(0.001, 0.01, n)
    out = torch.empty((m, n), dtype=torch.float64, device="cuda:0")
    from baracuda_amd.ffi import lib
    tw, ta, tsa, tsw = dev(w), dev(a), dev(sa), dev(sw)
    st = lib().quantized_linear_w8a8_f64_gfx950_run(m, n, k, tw.data_ptr(), ta.data_ptr(),
                                                    tsa.data_ptr(), tsw.data_ptr(), out.data_ptr(),
                                                    None, 0, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    sync()
    acc = O.gemm_s8_rcr_i32(a, w).astype(np.float32)
    want = ((sa.astype(np.float32)[:, None] * sw.astype(np.float32)[None, :]) * acc).astype(np.float64)
    got = out.cpu().numpy()
    assert np.array_equal(got, want)
    f64_product = (sa[:, None] * sw[None, :]) * acc.astype(np.float64)
    assert not np.array_equal(got, f64_product)     # the f32 evaluation is what is matched


def test_int8_determinism_replays(gpu):
    a, w, sa, sw = w8a8(1024, 768, 1024, seed=4)
    outs = [_w8a8(a, w, sa, sw) for _ in range(3)]
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


# ---- FP8 ---------------------------------------------------------------------
def _fp8_inputs(m, n, k, seed=3):
    # BASELINE.json config 3 recipe: N(0,1), scale absmax -> 448, cast to e4m3.
    g = rng(seed)
    xa = g.standard_normal((m, k)).astype(np.float32)
    xb = g.standard_normal((n, k)).astype(np.float32)
    sa = np.float32(np.abs(xa).max() / 448.0)
    sb = np.float32(np.abs(xb).max() / 448.0)
    ta = torch.from_numpy(xa / sa).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    tb = torch.from_numpy(xb / sb).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return ta, tb, float(sa), float(sb)


def _fp8_run(a, b, output, **kw):
    m, k = a.shape
    n = b.shape[0]
    dt = {P.ElementKind.F32: torch.float32, P.ElementKind.Bf16: torch.bfloat16, P.ElementKind.Fp8E4M3: torch.uint8}[output]
    d = torch.zeros((m, n), dtype=dt, device="cuda:0")
    P.Fp8GemmPlan.select(P.Fp8GemmDescriptor(m, n, k, output=output)).run(dev(a), dev(b), d, **kw)
    sync()
    return d


def _fp8_check_acc(got, a, b, alpha=1.0, rows=None):
    exact = O.gemm_fp8_e4m3_f64(a, b, rows=rows, nthreads=8) * alpha
    ta, tb = np.abs(O.e4m3_to_f32(a).astype(np.float64)), np.abs(O.e4m3_to_f32(b).astype(np.float64))
    absum = (ta[rows[0]:rows[1]] if rows else ta) @ tb.T * abs(alpha)
    err = np.abs(got.astype(np.float64) - exact)
    assert np.all(err <= 1e-3 * np.abs(exact) + FP8_FLOOR * absum), err.max()
    return exact


@pytest.mark.parametrize("shape", REF_SHAPES + [(512, 384, 1024)] + DMA_SHAPES[:4])
def test_fp8_f32_accumulator(gpu, shape):
    print(f"case: fp8 f32 {shape}", flush=True)
    a, b, _, _ = _fp8_inputs(*shape)
    got = _fp8_run(a, b, P.ElementKind.F32, alpha=1.0).cpu().numpy()
    _fp8_check_acc(got, a, b)


@pytest.mark.parametrize("shape", [(300, 520, 384), (1, 256, 4096), (257, 264, 128), (100, 68, 256)])
def test_fp8_edge_tiles_dma_path(gpu, shape):
    # f32 accumulators and bf16 outputs of edge tiles on the LDS-DMA path
    print(f"case: fp8 edge {shape}", flush=True)
    a, b, sa, sb = _fp8_inputs(*shape, seed=shape[0])
    got = _fp8_run(a, b, P.ElementKind.F32, alpha=1.0).cpu().numpy()
    exact = _fp8_check_acc(got, a, b)
    gotb = _fp8_run(a, b, P.ElementKind.Bf16, scale_a=sa, scale_b=sb).float().cpu().numpy().astype(np.float64)
    ta, tb = np.abs(O.e4m3_to_f32(a).astype(np.float64)), np.abs(O.e4m3_to_f32(b).astype(np.float64))
    want = exact * (np.float64(np.float32(sa) * np.float32(sb)))
    tol = bf16_ulp(want) + FP8_FLOOR * (ta @ tb.T) * float(np.float32(sa) * np.float32(sb))
    assert np.all(np.abs(gotb - want) <= tol)


def test_fp8_e4m3_out_reference_pattern(gpu):
    # fp8_e4m3_rcr_smoke.rs:113-126 patterns, alpha = 0.25; +-1 e4m3 grid step.
    for (m, n, k) in REF_SHAPES + [(256, 256, 128)]:
        a = O.f32_to_e4m3((((np.arange(m * k) * 5) % 13) - 6.0) * 0.125).reshape(m, k)
        b = O.f32_to_e4m3((((np.arange(k * n) * 7) % 11) - 5.0) * 0.125).reshape(n, k)
        got = O.e4m3_to_f32(_fp8_run(a, b, P.ElementKind.Fp8E4M3, alpha=0.25).cpu().numpy())
        # the patterns are small dyadic rationals: the f32 sum is exact, so the
        # e4m3 output must equal the oracle's encode of the exact value.
        want = O.e4m3_to_f32(O.f32_to_e4m3((O.gemm_fp8_e4m3_f64(a, b) * 0.25).astype(np.float32)))
        assert np.array_equal(got, want), (m, n, k)


def test_fp8_bf16_config3_sampled(gpu):
    # BASELINE.json config 3 at full size.  Per element, 32 sampled rows (4 in
    # each of the 8 tile-rows of 256, at varying offsets; every row crosses
    # all 56 tile-columns, so both rounds of the 448-tile grid) against the
    # f64 oracle within 1 bf16 ulp + FP8_FLOOR_CONFIG3 * sum|a*b|.  Over the whole
    # 2048 x 14336 output:
    #   - the f32-out SKU against the exact f64 product (a GPU f64 matmul of
    #     the decoded operands) and against hipBLASLt (torch._scaled_mm, an independent
    #     library on the same operands) within 1e-3 rel + FP8_FLOOR_CONFIG3 * sum|a*b|;
    #   - the bf16-out SKU equals bf16_rne(alpha * f32-out) bit for bit (both
    #     SKUs share the mainloop, so this pins the bf16 epilogue everywhere);
    #   - every row sum of the f32 output against the exact f64
    #     sum_k dec(a[m,k]) * sum_n dec(b[n,k]), within the summed per-element bound.
    print("case: fp8 bf16 2048x14336x4096", flush=True)
    m, n, k = 2048, 14336, 4096
    a, b, sa, sb = _fp8_inputs(m, n, k)
    d = _fp8_run(a, b, P.ElementKind.Bf16, scale_a=sa, scale_b=sb)
    got = O.bf16_bits_to_f32(host_bits16(d))
    alpha = float(np.float32(sa) * np.float32(sb))
    fa = O.e4m3_to_f32(a).astype(np.float64)
    fb = O.e4m3_to_f32(b).astype(np.float64)
    abs_b = np.abs(fb)
    rows = sorted({t * 256 + off for t in range(8) for off in (0, 37 + 19 * t, 128 + 7 * t, 255)})
    assert len(rows) == 32
    for r in rows:
        exact = O.gemm_fp8_e4m3_f64(a, b, rows=(r, r + 1), nthreads=8)[0] * alpha
        err = np.abs(got[r].astype(np.float64) - exact)
        absum = abs_b @ np.abs(fa[r]) * alpha
        assert np.all(err <= bf16_ulp(exact) + FP8_FLOOR_CONFIG3 * absum), (r, err.max())
    del d, got
    f32 = _fp8_run(a, b, P.ElementKind.F32, alpha=1.0)
    one = torch.tensor(1.0, device="cuda:0")
    ref = torch._scaled_mm(dev(a).view(torch.float8_e4m3fn), dev(b).view(torch.float8_e4m3fn).t(),
                           scale_a=one, scale_b=one, out_dtype=torch.float32)
    ours = f32.cpu().numpy()
    ref = ref.cpu().numpy().astype(np.float64)
    absum = torch.from_numpy(np.abs(fa)).cuda() @ torch.from_numpy(abs_b).cuda().T   # f64 on the GPU
    absum = absum.cpu().numpy()
    # the f64 product of the decoded operands: its rounding (< 2^-40 * sum|a*b|
    # for K = 4096) is far below the bar
    exact = (torch.from_numpy(fa).cuda() @ torch.from_numpy(fb).cuda().T).cpu().numpy()
    assert np.all(np.abs(ours.astype(np.float64) - exact) <= 1e-3 * np.abs(exact) + FP8_FLOOR_CONFIG3 * absum)
    del exact
    assert np.all(np.abs(ours.astype(np.float64) - ref) <= 1e-3 * np.abs(ref) + FP8_FLOOR_CONFIG3 * absum)
    bf = host_bits16(_fp8_run(a, b, P.ElementKind.Bf16, scale_a=sa, scale_b=sb))
    assert np.array_equal(bf, O.f32_to_bf16_bits_fast(np.float32(alpha) * ours))
    row_exact = fa @ fb.sum(0)                       # sum_n sum_k a b, exact in f64
    row_tol = (1e-3 * np.abs(ref) + FP8_FLOOR_CONFIG3 * absum).sum(1)
    assert np.all(np.abs(ours.astype(np.float64).sum(1) - row_exact) <= row_tol)


@pytest.mark.parametrize("shape", [(256, 128, 64), (512, 512, 1024), (256, 512, 384)])
def test_fp8_matches_hipblaslt(gpu, shape):
    # Independent library cross-check: hipBLASLt's FP8 GEMM (torch._scaled_mm) on
    # the same e4m3 operands, f32 out; both run the same MFMA instruction.
    m, n, k = shape
    a, b, _, _ = _fp8_inputs(m, n, k)
    ours = _fp8_run(a, b, P.ElementKind.F32, alpha=1.0).cpu().numpy().astype(np.float64)
    ta = dev(a).view(torch.float8_e4m3fn)
    tb = dev(b).view(torch.float8_e4m3fn)
    one = torch.tensor(1.0, device="cuda:0")
    ref = torch._scaled_mm(ta, tb.t(), scale_a=one, scale_b=one, out_dtype=torch.float32)
    sync()
    ref = ref.cpu().numpy().astype(np.float64)
    absum = np.abs(O.e4m3_to_f32(a).astype(np.float64)) @ np.abs(O.e4m3_to_f32(b).astype(np.float64)).T
    assert np.all(np.abs(ours - ref) <= 1e-3 * np.abs(ref) + FP8_FLOOR * absum)


# ---- per-token dynamic quantization + the W8A8 pipeline ------------------------
def _quant_gpu(x, dtype, qmin=-127, qmax=127):
    from baracuda_amd.ffi import lib
    n, dd = x.shape
    tx = torch.from_numpy(x).to(dtype).cuda()
    sdt = torch.float32 if dtype == torch.bfloat16 else dtype
    scale = torch.zeros(n, dtype=sdt, device="cuda:0")
    q = torch.zeros((n, dd), dtype=torch.int8, device="cuda:0")
    L = lib()
    fn = {torch.float32: L.dynamic_range_quantize_per_token_sym_f32_s8_run,
          torch.float64: L.dynamic_range_quantize_per_token_sym_f64_s8_run,
          torch.bfloat16: L.dynamic_range_quantize_per_token_sym_bf16_s8_gfx950_run}[dtype]
    st = fn(n, dd, qmin, qmax, tx.data_ptr(), scale.data_ptr(), q.data_ptr(), None, 0,
            torch.cuda.current_stream().cuda_stream)
    assert st == 0
    sync()
    # the value the kernel reads, as f32 (qc_load_as_f32)
    seen = tx.float().cpu().numpy()
    return q.cpu().numpy(), scale.cpu().numpy(), seen


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
@pytest.mark.parametrize("shape", [(64, 4096), (7, 333), (3, 20000), (1, 1), (5, 16384), (9, 24), (6, 8192),
                                   (5, 8200), (13, 8), (4, 2048), (4, 2056), (4, 4104), (5, 4096), (3, 4088),
                                   (10, 520), (6, 1032), (7, 512), (9, 1024)])
def test_quantize_per_token_bit_exact(gpu, dtype, shape):
    print(f"case: quantize {dtype} {shape}", flush=True)
    g = rng(shape[0] * 31 + shape[1])
    x = (g.standard_normal(shape) * 10 ** g.uniform(-2, 2, (shape[0], 1))).astype(np.float64)
    if shape[0] > 3:
        x[2] = 0.0
    q, s, seen = _quant_gpu(x, dtype)
    wq, ws = O.quantize_per_token_sym(seen)
    assert np.array_equal(q, wq)
    assert np.array_equal(s.astype(np.float32), ws)


def test_quantize_many_rows_grid_stride(gpu):
    # N above the 65535-workgroup grid: rows are grid-strided.
    x = rng(5).standard_normal((70000, 16)).astype(np.float32)
    for dt in (torch.float32, torch.bfloat16):   # scalar and 16-byte-chunk paths
        q, s, seen = _quant_gpu(x, dt, -128, 127)
        wq, ws = O.quantize_per_token_sym(seen, -128, 127)
        assert np.array_equal(q, wq) and np.array_equal(s.astype(np.float32), ws)


def test_quantize_bf16_rows_grid_stride(gpu):
    # bf16 16-byte-chunk path with N far above the 65535-workgroup grid.
    x = rng(6).standard_normal((270001, 8)).astype(np.float32)
    q, s, seen = _quant_gpu(x, torch.bfloat16)
    wq, ws = O.quantize_per_token_sym(seen)
    assert np.array_equal(q, wq) and np.array_equal(s.astype(np.float32), ws)


def test_quantize_then_w8a8_matches_fp_matmul(gpu):
    # quantized_linear_smoke.rs: quantize activations per token, weights per
    # channel, W8A8 GEMM; compare with the fp32 matmul (~2% relative).
    g = rng(23)
    m, n, k = 256, 512, 1024
    a = g.standard_normal((m, k)).astype(np.float32)
    w = (g.standard_normal((n, k)) * 0.05).astype(np.float32)
    wq, ws = O.quantize_per_token_sym(w)          # per-output-channel symmetric
    aq, sa, _ = _quant_gpu(a, torch.float32)
    d = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16)).run(
        dev(aq), dev(wq), d, scale_a=dev(sa), scale_b=dev(ws))
    sync()
    got = O.bf16_bits_to_f32(host_bits16(d)).astype(np.float64)
    ref = a.astype(np.float64) @ w.astype(np.float64).T
    err = np.abs(got - ref)
    assert err.max() <= 0.02 * np.abs(ref).max()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
def test_quantized_linear_plan_two_pass(gpu, dtype):
    # QuantizedLinearPlan::run = quantize (pass 1) + W8A8 GEMM (pass 2); the
    # output equals the oracle chain on the same activation.
    g = rng(29)
    m, c_out, k = 96, 256, 512
    a = g.standard_normal((m, k)).astype(np.float32)
    wq, ws = O.quantize_per_token_sym((g.standard_normal((c_out, k)) * 0.1).astype(np.float32))
    ta = torch.from_numpy(a).to(dtype).cuda()
    out = torch.empty((m, c_out), dtype=dtype, device="cuda:0")
    aq = torch.empty((m, k), dtype=torch.int8, device="cuda:0")
    sdt = torch.float64 if dtype == torch.float64 else torch.float32
    sa = torch.empty(m, dtype=sdt, device="cuda:0")
    plan = P.QuantizedLinearPlan.select(P.QuantizedLinearDescriptor(m, c_out, k))
    plan.run(ta, dev(wq), dev(ws).to(sdt), out, aq, sa)
    sync()
    # f64 activations are read through an f32 narrowing (the reference's
    # qc_load_as_f32), so the oracle chain runs on the f32 values throughout.
    qa, sa_ref = O.quantize_per_token_sym(ta.float().cpu().numpy())
    assert np.array_equal(aq.cpu().numpy(), qa) and np.array_equal(sa.cpu().numpy(), sa_ref)
    acc = O.gemm_s8_rcr_i32(qa, wq).astype(np.float32)
    want = (sa_ref[:, None] * ws[None, :]).astype(np.float32) * acc
    if dtype == torch.float32:
        assert np.array_equal(out.cpu().numpy(), want)
    elif dtype == torch.float64:
        assert np.array_equal(out.cpu().numpy(), want.astype(np.float64))
    else:
        assert np.array_equal(host_bits16(out), O.f32_to_bf16_bits_fast(want))


def test_i32_operand_beyond_2gib(gpu):
    # A is 16384 x 131200 int8 (2.0 GiB): past the 32-bit buffer offsets of
    # the LDS-DMA path, so the general kernel (64-bit row addressing) runs.
    # Sampled rows are compared exactly against an int64 dot product.
    m, n, k = 16384, 256, 131200
    print(f"case: i32 beyond 2 GiB {m}x{n}x{k}", flush=True)
    gen = torch.Generator(device="cuda:0").manual_seed(77)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device="cuda:0", generator=gen)
    b = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda:0", generator=gen)
    assert m * k >= 2 ** 31
    d = torch.empty((m, n), dtype=torch.int32, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.I32)).run(a, b, d)
    sync()
    rows = [0, 1, 8191, 16383] + list(rng(78).integers(0, m, 4))
    bh = b.cpu().numpy().astype(np.int64)
    got = d[rows].cpu().numpy()
    for i, r in enumerate(rows):
        want = bh @ a[r].cpu().numpy().astype(np.int64)
        assert np.array_equal(got[i], want.astype(np.int32)), r
    del a


@pytest.mark.parametrize("n, dd", [(131080, 16384), (524290, 4096)])
def test_quantize_bf16_input_beyond_2gib(gpu, n, dd):
    # 2^31 + 131072 / 8192 elements (4 GiB of input, 2 GiB of int8 output),
    # so element indices and byte offsets pass 2^31: 64-bit row offsets in
    # the 16-byte-chunk paths (a workgroup per row for D = 16384, a wave per
    # row for D = 4096); sampled rows (the last lie wholly past element
    # 2^31) bit-exact.
    assert n * dd > 2 ** 31
    print(f"case: quantize beyond 2^31 elements {n}x{dd}", flush=True)
    gen = torch.Generator(device="cuda:0").manual_seed(93)
    x = torch.empty((n, dd), device="cuda:0", dtype=torch.bfloat16)
    x.normal_(generator=gen)
    q = torch.empty((n, dd), dtype=torch.int8, device="cuda:0")
    scale = torch.empty(n, dtype=torch.float32, device="cuda:0")
    P.dynamic_range_quantize_per_token_sym(x, scale, q)
    sync()
    first_past = 2 ** 31 // dd
    rows = [0, 1, 65535, first_past - 1, first_past, min(first_past + 3, n - 1), n - 1]
    rows += list(rng(94).integers(0, n, 4))
    # rows read through basic-index views (x[r]), which raise on an index
    # past N on the host instead of handing it to a device gather
    seen = np.stack([x[int(r)].float().cpu().numpy() for r in rows])
    wq, ws = O.quantize_per_token_sym(seen)
    assert np.array_equal(np.stack([q[int(r)].cpu().numpy() for r in rows]), wq)
    assert np.array_equal(np.array([scale[int(r)].item() for r in rows], dtype=np.float32), ws)
    del x, q
