"""GPU parity of the FP8 RCR last-rows pass (gemm_fp8_rcr_rows_staged_kernel,
and gemm_fp8_rcr_row1_kernel for one row): decode-sized M (all of it) and
the last M % 256 rows when a row of tiles would start another round, for
every stage shape the launcher picks (fragments x columns per workgroup and
stage bytes) and the fall-backs when N or K does not divide the preferred
one.

The reference smoke pattern (fp8_bias_smoke.rs inputs: small dyadic values
whose f32 partial sums are exact in any order) must come out bit-exact for
Identity / Bias / BiasRelu and within one grid step for BiasGelu / BiasSilu,
as on the tile path; random N(0,1) operands keep the tile path's tolerance
(1e-3 relative + FP8_FLOOR * sum|a*b| for f32 accumulators, one bf16 ulp plus
that floor for bf16 outputs).
"""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from oracle import oracle as O
from tests.gpu_util import FP8_FLOOR, bf16_ulp, dev, sync
from tests.test_gpu_fp8_epi import EPIS, ACT, _run, _steps, _want
from tests.test_gpu_gemm import _fp8_check_acc, _fp8_inputs, _fp8_run

pytestmark = pytest.mark.gpu

# (M, N, K) and the stage shape they take: 16 columns per workgroup below
# N = 6144 (1 fragment with 2 KiB stages: 1 / 16, K % 2048 == 0; 2 with
# 1 KiB: 5 with K % 2048 != 0, 17, 32; 4 with 512 B: 9 and 20 with
# K % 1024 != 0, 33, 64; 8: 65, 100, 128), 32 columns from N = 6144 (2 / 33
# with 4 fragments, 128 with 8), 64 columns from N = 12288 (1 / 16 with 4
# fragments, 100 with 8 and 256-byte stages).  Under 4 tile rows at
# N = 16384 (the tiles fill one round exactly): 1 / 40 / 128 last rows.
# 129-512 rows whose row blocks fit one round of workgroups: every row as
# blocks of the same kernel (64-row blocks at 200 / 384, 128-row blocks at
# 512 x 4096).  One row with K % 1024 == 0
# (1 x 256 / 1040 / 12288 / 512, 1025 x 16384) takes the FMA row kernel
# instead (2 KiB per batch, 1 KiB at K = 3072).  33-128 rows below N = 6144
# with K % 1024 == 0 run as row blocks: 64-row blocks of 32 / 16 columns
# (100 x 4096, 90 x 2560), 32-row blocks with 1 KiB stages (60 x 3072,
# 100 x 512).  From N = 6144 up to 16 / 32 rows take 1 / 2 fragments with
# only 4 / 8 waves multiplying (9 x 8192, 16 x 14336, 20 x 8192, 30 x 14336;
# 2 x 6144).
SHAPES = [(1, 256, 4096), (16, 512, 2048), (5, 272, 1024), (17, 288, 1024), (32, 1040, 3072),
          (9, 256, 1536), (20, 272, 512), (33, 512, 512), (64, 256, 2560), (65, 1040, 1024),
          (100, 512, 4096), (128, 256, 512), (1025, 16384, 2048), (1064, 16384, 512), (1152, 16384, 1024),
          (1, 1040, 4096), (16, 272, 2048), (2, 6144, 512), (33, 8192, 512), (128, 6144, 1024),
          (1, 12288, 2048), (16, 14336, 1024), (100, 12288, 1024), (200, 512, 1024), (384, 1024, 512),
          (512, 4096, 512), (1, 512, 3072), (100, 4096, 1024), (60, 3072, 1024), (90, 2560, 1024),
          (20, 8192, 1024), (30, 14336, 512), (9, 8192, 512)]


@pytest.mark.parametrize("shape", SHAPES)
def test_fp8_rows_f32_and_bf16(gpu, shape):
    m, n, k = shape
    print(f"case: fp8 rows f32/bf16 {shape}", flush=True)
    a, b, sa, sb = _fp8_inputs(m, n, k, seed=m + n + k)
    rows = (max(0, m - m % 256 - 2), m) if m > 256 else None
    got = _fp8_run(a, b, P.ElementKind.F32, alpha=1.0).cpu().numpy()
    exact = _fp8_check_acc(got[rows[0]:rows[1]] if rows else got, a, b, rows=rows)
    gotb = _fp8_run(a, b, P.ElementKind.Bf16, scale_a=sa, scale_b=sb).float().cpu().numpy().astype(np.float64)
    if rows:
        gotb = gotb[rows[0]:rows[1]]
    ta = np.abs(O.e4m3_to_f32(a).astype(np.float64))
    tb = np.abs(O.e4m3_to_f32(b).astype(np.float64))
    s = float(np.float32(sa) * np.float32(sb))
    want = exact * s
    tol = bf16_ulp(want) + FP8_FLOOR * ((ta[rows[0]:rows[1]] if rows else ta) @ tb.T) * s
    assert np.all(np.abs(gotb - want) <= tol)


@pytest.mark.parametrize("epi", EPIS)
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape", [SHAPES[0], SHAPES[3], SHAPES[7], SHAPES[10], SHAPES[13], SHAPES[15], SHAPES[18], SHAPES[22], SHAPES[23], SHAPES[25], SHAPES[26], SHAPES[27], SHAPES[28], SHAPES[30], SHAPES[31], SHAPES[32]])
def test_fp8_rows_reference_pattern(gpu, shape, fmt, epi):
    m, n, k = shape
    print(f"case: fp8 rows pattern {fmt} {epi.value} {shape}", flush=True)
    a = O.f32_to_fp8((((np.arange(m * k) * 5) % 13) - 6.0) * 0.125, fmt).reshape(m, k)
    b = O.f32_to_fp8((((np.arange(k * n) * 7) % 11) - 5.0) * 0.125, fmt).reshape(n, k)
    bias = (((np.arange(n) % 5) - 2) * 0.5).astype(np.float32)
    got = _run(fmt, P.LayoutSku.Rcr, epi, a, b, bias=bias)
    want = _want(fmt, P.LayoutSku.Rcr, epi, a, b, None, bias, 0.25, 0.0)
    if ACT[epi] in (None, "relu"):
        assert np.array_equal(got, want)
    else:
        assert _steps(got, want, fmt).max() <= 1.0


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape", [SHAPES[1], SHAPES[4], SHAPES[9], SHAPES[14], SHAPES[16], SHAPES[19], SHAPES[21], SHAPES[24], SHAPES[29], SHAPES[10]])
def test_fp8_rows_random_with_c(gpu, shape, fmt):
    # C (beta = 0.5) and a BiasGelu epilogue on random operands: one grid step
    # plus the MFMA's summation floor, as the tile path's test.
    m, n, k = shape
    print(f"case: fp8 rows random with C {fmt} {shape}", flush=True)
    g = np.random.default_rng(m * 7 + n + k)
    a = O.f32_to_fp8(g.standard_normal((m, k)).astype(np.float32), fmt)
    b = O.f32_to_fp8(g.standard_normal((n, k)).astype(np.float32), fmt)
    c = O.f32_to_fp8(g.standard_normal((m, n)).astype(np.float32), fmt)
    bias = g.standard_normal(n).astype(np.float32)
    alpha = 1.0 / 16
    epi = P.EpilogueKind.BiasGelu
    got = _run(fmt, P.LayoutSku.Rcr, epi, a, b, c=c, bias=bias, alpha=alpha, beta=0.5)
    want = _want(fmt, P.LayoutSku.Rcr, epi, a, b, c, bias, alpha, 0.5)
    fa = np.abs(O.fp8_to_f32(a, fmt).astype(np.float64))
    fb = np.abs(O.fp8_to_f32(b, fmt).astype(np.float64))
    st = _steps(got, want, fmt, FP8_FLOOR * alpha * (fa @ fb.T))
    assert st.max() <= 1.0 and (got != want).mean() < 0.02


def test_fp8_rows_deterministic_and_untouched_columns(gpu):
    # Repeated calls give identical bits (fixed chunk order); D columns and
    # rows outside the problem (a wider, taller buffer) are not written.
    m, n, k = 40, 512, 2048
    a, b, sa, sb = _fp8_inputs(m, n, k, seed=11)
    plan = P.Fp8GemmPlan.select(P.Fp8GemmDescriptor(m, n, k, output=P.ElementKind.Bf16))
    outs = []
    for _ in range(3):
        big = torch.full((m + 3, n + 64), -7.0, dtype=torch.bfloat16, device="cuda:0")
        plan.run(dev(a), dev(b), big[:m, :n], scale_a=sa, scale_b=sb)
        sync()
        h = big.float().cpu().numpy()
        assert np.all(h[:, n:] == -7.0) and np.all(h[m:, :] == -7.0)
        outs.append(h[:m, :n])
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


# RRR (row-major B [K, N]) last rows: the staged kernel with transposing LDS
# reads; 16 / 32 / 64 columns per workgroup by the last-rows rule, 1 / 2 / 4 /
# 8 fragments, main RRR tiles above the rows at N = 16384; row blocks below
# N = 6144 with K % 1024 == 0 (100 x 512, 100 x 4096, 60 x 3072); up to 16 /
# 32 rows on 1 / 2 fragments with only some waves multiplying (1 x 256,
# 5 x 272, 9 x 14336, 17 x 6144, 30 x 14336).
RRR_SHAPES = [(1, 256, 4096), (17, 288, 1024), (33, 272, 512), (5, 272, 2048), (100, 512, 1024),
              (128, 1040, 512), (1025, 16384, 512), (17, 6144, 1024), (64, 8192, 512),
              (100, 4096, 1024), (60, 3072, 1024), (9, 14336, 512), (30, 14336, 1024)]


@pytest.mark.parametrize("epi", EPIS)
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape", RRR_SHAPES)
def test_fp8_rrr_rows_reference_pattern(gpu, shape, fmt, epi):
    m, n, k = shape
    print(f"case: fp8 rrr rows pattern {fmt} {epi.value} {shape}", flush=True)
    a = O.f32_to_fp8((((np.arange(m * k) * 5) % 13) - 6.0) * 0.125, fmt).reshape(m, k)
    b = O.f32_to_fp8((((np.arange(k * n) * 7) % 11) - 5.0) * 0.125, fmt).reshape(k, n)
    bias = (((np.arange(n) % 5) - 2) * 0.5).astype(np.float32)
    got = _run(fmt, P.LayoutSku.Rrr, epi, a, b, bias=bias)
    rows = slice(max(0, m - m % 256 - 2), m) if m > 256 else slice(0, m)
    want = _want(fmt, P.LayoutSku.Rrr, epi, a[rows], b, None, bias, 0.25, 0.0)
    if ACT[epi] in (None, "relu"):
        assert np.array_equal(got[rows], want)
    else:
        assert _steps(got[rows], want, fmt).max() <= 1.0


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape", [RRR_SHAPES[1], RRR_SHAPES[3], RRR_SHAPES[4]])
def test_fp8_rrr_rows_random_with_c(gpu, shape, fmt):
    m, n, k = shape
    print(f"case: fp8 rrr rows random with C {fmt} {shape}", flush=True)
    g = np.random.default_rng(m * 11 + n + k)
    a = O.f32_to_fp8(g.standard_normal((m, k)).astype(np.float32), fmt)
    b = O.f32_to_fp8(g.standard_normal((k, n)).astype(np.float32), fmt)
    c = O.f32_to_fp8(g.standard_normal((m, n)).astype(np.float32), fmt)
    bias = g.standard_normal(n).astype(np.float32)
    alpha = 1.0 / 16
    epi = P.EpilogueKind.BiasSilu
    got = _run(fmt, P.LayoutSku.Rrr, epi, a, b, c=c, bias=bias, alpha=alpha, beta=0.5)
    want = _want(fmt, P.LayoutSku.Rrr, epi, a, b, c, bias, alpha, 0.5)
    fa = np.abs(O.fp8_to_f32(a, fmt).astype(np.float64))
    fb = np.abs(O.fp8_to_f32(b, fmt).astype(np.float64))
    st = _steps(got, want, fmt, FP8_FLOOR * alpha * (fa @ fb))
    assert st.max() <= 1.0 and (got != want).mean() < 0.02


# FP8 RRR small grids (129-512 rows): every row as row blocks of the staged
# kernel with row-major B: 64-row blocks at 200 x 512, 128-row blocks at
# 512 x 4096 and 300 x 1024, where 64-row blocks would need a second round.
@pytest.mark.parametrize("epi", [P.EpilogueKind.Identity, P.EpilogueKind.BiasGelu])
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape", [(200, 512, 1024), (512, 4096, 512), (300, 1024, 512)])
def test_fp8_rrr_small_grid_row_blocks(gpu, shape, fmt, epi):
    m, n, k = shape
    print(f"case: fp8 rrr small grid {fmt} {epi.value} {shape}", flush=True)
    a = O.f32_to_fp8((((np.arange(m * k) * 5) % 13) - 6.0) * 0.125, fmt).reshape(m, k)
    b = O.f32_to_fp8((((np.arange(k * n) * 7) % 11) - 5.0) * 0.125, fmt).reshape(k, n)
    bias = (((np.arange(n) % 5) - 2) * 0.5).astype(np.float32)
    got = _run(fmt, P.LayoutSku.Rrr, epi, a, b, bias=bias)
    want = _want(fmt, P.LayoutSku.Rrr, epi, a, b, None, bias, 0.25, 0.0)
    if ACT[epi] in (None, "relu"):
        assert np.array_equal(got, want)
    else:
        assert _steps(got, want, fmt).max() <= 1.0


@pytest.mark.parametrize("shape", [(1, 4096, 2048), (16, 14336, 1024), (100, 4096, 1024), (256, 4096, 512)])
def test_fp8_rows_padded_leading_dimensions(gpu, shape):
    # A, B and D views with pitches past K / N: the one-row kernel, the
    # partial-wave blocks, the row blocks and a small grid's blocks address
    # rows by lda / ldb / ldd; f32 accumulators against the f64 sum, columns
    # past N untouched.
    m, n, k = shape
    print(f"case: fp8 rows padded ld {shape}", flush=True)
    a, b, _, _ = _fp8_inputs(m, n, k, seed=m + 2 * n + k)
    a_full = np.zeros((m, k + 64), np.uint8)
    b_full = np.zeros((n, k + 128), np.uint8)
    a_full[:, :k], b_full[:, :k] = a, b
    d_full = torch.full((m, n + 32), -7.0, dtype=torch.float32, device="cuda:0")
    P.Fp8GemmPlan.select(P.Fp8GemmDescriptor(m, n, k, output=P.ElementKind.F32)).run(
        dev(a_full)[:, :k], dev(b_full)[:, :k], d_full[:, :n], alpha=1.0)
    sync()
    got = d_full.cpu().numpy()
    _fp8_check_acc(got[:, :n], a, b)
    assert np.all(got[:, n:] == -7.0)
