"""GPU parity of the int8 RRR GEMM, the u8 RRR and RCR GEMMs and the bias /
activation epilogue family (RCR and RRR) against the CPU oracle.

Inputs follow the reference smoke test (crates/baracuda-kernels/tests/
int8_rrr_smoke.rs): a = ((7i)%15)-7, b = ((11i)%13)-6, alpha = 0.125, bias
f32 ((j%5)-2)*0.5 or i32 ((j%5)-2)*2, plus seeded random operands with C.
Bars, as in that test: Identity / Bias / BiasRelu bit-exact; BiasGelu /
BiasSilu within 1 int8 step (the GPU evaluates the same Abramowitz-Stegun erf
as the reference CPU side, but with the hardware exp / reciprocal), with
off-by-one results on under 1% of the outputs.
"""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from oracle import oracle as O
from oracle.inputs import int8_uniform, rng
from tests.gpu_util import dev, sync

pytestmark = pytest.mark.gpu

EPIS = [P.EpilogueKind.Identity, P.EpilogueKind.Bias, P.EpilogueKind.BiasRelu,
        P.EpilogueKind.BiasGelu, P.EpilogueKind.BiasSilu]
ACT = {P.EpilogueKind.Identity: None, P.EpilogueKind.Bias: None, P.EpilogueKind.BiasRelu: "relu",
       P.EpilogueKind.BiasGelu: "gelu", P.EpilogueKind.BiasSilu: "silu"}
REF_SHAPES = [(64, 64, 32), (128, 128, 128), (256, 128, 64), (100, 70, 50)]
# Aligned RRR / LDS-DMA RCR shapes (whole 256x256 tiles, K % 128 == 0) and ragged ones.
BIG_SHAPES = [(256, 256, 128), (512, 768, 384), (300, 520, 200), (1, 256, 4096)]


def _pattern(m, n, k, layout):
    a = ((np.arange(m * k) * 7) % 15 - 7).astype(np.int8).reshape(m, k)
    b = ((np.arange(k * n) * 11) % 13 - 6).astype(np.int8)
    b = b.reshape(k, n) if layout == P.LayoutSku.Rrr else b.reshape(n, k)
    return a, b


def _bias(n, kind):
    j = np.arange(n)
    if kind == P.ElementKind.F32:
        return (((j % 5) - 2) * 0.5).astype(np.float32)
    return (((j % 5) - 2) * 2).astype(np.int32)


def _run(layout, epi, bias_kind, a, b, c=None, bias=None, alpha=0.125, beta=0.0):
    m, k = a.shape
    n = b.shape[1] if layout == P.LayoutSku.Rrr else b.shape[0]
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, layout=layout, epilogue=epi,
                                                    bias_element=bias_kind))
    d = torch.full((m, n), 99, dtype=torch.int8, device="cuda:0")
    plan.run(dev(a), dev(b), d, c=None if c is None else dev(c), alpha=alpha, beta=beta,
             bias=None if bias is None else dev(bias))
    sync()
    return d.cpu().numpy()


def _want(layout, epi, a, b, c, bias, alpha, beta):
    return O.gemm_s8_epi(a, b, "rrr" if layout == P.LayoutSku.Rrr else "rcr", alpha, beta, c,
                         None if epi == P.EpilogueKind.Identity else bias, ACT[epi])


def _check(got, want, epi):
    diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
    if ACT[epi] in (None, "relu"):
        assert diff.max() == 0, f"max diff {diff.max()} at {np.argwhere(diff)[:4]}"
    else:
        assert diff.max() <= 1 and (diff != 0).mean() < 0.01


@pytest.mark.parametrize("epi", [P.EpilogueKind.Identity, P.EpilogueKind.BiasRelu])
@pytest.mark.parametrize("layout", [P.LayoutSku.Rrr, P.LayoutSku.Rcr])
@pytest.mark.parametrize("shape", [(300, 528, 384), (1, 256, 4096), (257, 272, 128), (100, 68, 256)])
def test_edge_tiles_dma_path_with_c(gpu, shape, layout, epi):
    # K % 128 == 0 with M / N off the 256 grid: the LDS-DMA kernels with
    # zero-filled rows past M (and RRR B columns past N) and masked stores.
    m, n, k = shape
    print(f"case: edge {layout.value} {epi.value} {shape}", flush=True)
    g = rng(m + 5 * n + 7 * k)
    a = int8_uniform(g, (m, k))
    b = int8_uniform(g, (k, n) if layout == P.LayoutSku.Rrr else (n, k))
    c = int8_uniform(g, (m, n))
    bias = (g.standard_normal(n) * 8).astype(np.float32)
    got = _run(layout, epi, P.ElementKind.F32, a, b, c=c, bias=bias, alpha=1.0 / 256, beta=0.75)
    _check(got, _want(layout, epi, a, b, c, bias, 1.0 / 256, 0.75), epi)


@pytest.mark.parametrize("bias_kind", [P.ElementKind.F32, P.ElementKind.I32])
@pytest.mark.parametrize("epi", EPIS)
@pytest.mark.parametrize("layout", [P.LayoutSku.Rrr, P.LayoutSku.Rcr])
@pytest.mark.parametrize("shape", REF_SHAPES)
def test_reference_smoke_pattern(gpu, shape, layout, epi, bias_kind):
    if epi == P.EpilogueKind.Identity and bias_kind == P.ElementKind.I32:
        pytest.skip("Identity has no bias")
    m, n, k = shape
    print(f"case: {layout.value} {epi.value} {bias_kind.value} {shape}", flush=True)
    a, b = _pattern(m, n, k, layout)
    bias = _bias(n, bias_kind)
    got = _run(layout, epi, bias_kind, a, b, bias=bias)
    _check(got, _want(layout, epi, a, b, None, bias, 0.125, 0.0), epi)


@pytest.mark.parametrize("epi", EPIS)
@pytest.mark.parametrize("layout", [P.LayoutSku.Rrr, P.LayoutSku.Rcr])
@pytest.mark.parametrize("shape", BIG_SHAPES)
def test_random_with_c(gpu, shape, layout, epi):
    m, n, k = shape
    print(f"case: random {layout.value} {epi.value} {shape}", flush=True)
    g = rng(m + 3 * n + 7 * k)
    a = int8_uniform(g, (m, k))
    b = int8_uniform(g, (k, n) if layout == P.LayoutSku.Rrr else (n, k))
    c = int8_uniform(g, (m, n))
    bias = (g.standard_normal(n) * 8).astype(np.float32)
    alpha = 1.0 / 256   # keeps z inside the int8 range so the activation shape matters
    got = _run(layout, epi, P.ElementKind.F32, a, b, c=c, bias=bias, alpha=alpha, beta=0.75)
    _check(got, _want(layout, epi, a, b, c, bias, alpha, 0.75), epi)


def test_rrr_strided_and_unaligned_operands(gpu):
    # Views with padded leading dimensions and a B base offset by 1 byte take
    # the checked (byte-granular) B path.
    m, n, k = 130, 260, 96
    g = rng(5)
    a_full = int8_uniform(g, (m, k + 16))
    b_full = int8_uniform(g, (k, n + 9))
    a_t, b_t = dev(a_full)[:, :k], dev(b_full)[:, 1:n + 1]
    d_full = torch.zeros((m, n + 4), dtype=torch.int8, device="cuda:0")
    d = d_full[:, :n]
    bias = _bias(n, P.ElementKind.I32)
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, layout=P.LayoutSku.Rrr,
                                                    epilogue=P.EpilogueKind.BiasRelu,
                                                    bias_element=P.ElementKind.I32))
    plan.run(a_t, b_t, d, alpha=0.125, bias=dev(bias))
    sync()
    want = O.gemm_s8_epi(a_full[:, :k], b_full[:, 1:n + 1], "rrr", 0.125, bias=bias, act="relu")
    assert np.array_equal(d.cpu().numpy(), want)
    assert np.all(d_full[:, n:].cpu().numpy() == 0)   # padding untouched


def test_rrr_large_k_sum_identity(gpu):
    # 2048 x 2048 x 4096 RRR Identity with alpha=1/4096: the full result
    # against torch's int64 matmul on the host, every 97th row against the oracle.
    m = n = 2048
    k = 4096
    g = rng(77)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (k, n))
    print("case: rrr identity 2048x2048x4096", flush=True)
    got = _run(P.LayoutSku.Rrr, P.EpilogueKind.Identity, P.ElementKind.F32, a, b, alpha=1.0 / 4096)
    ta, tb = torch.from_numpy(a).to(torch.int64), torch.from_numpy(b).to(torch.int64)
    acc = (ta @ tb).numpy().astype(np.float32)
    want = np.clip(np.rint(np.float32(1.0 / 4096) * acc), -128, 127).astype(np.int8)
    assert np.array_equal(got, want)
    rows = np.arange(0, m, 97)
    assert np.array_equal(got[rows], O.gemm_s8_epi(a[rows], b, "rrr", 1.0 / 4096))


# ---- U8 RRR and RCR (int8_rrr_smoke.rs / int8_smoke.rs run_u8_smoke:
# a = (7i)%16, b = (11i)%14) ---------------------------------------------------
RRR, RCR = P.LayoutSku.Rrr, P.LayoutSku.Rcr


def _run_u8(epi, bias_kind, a, b, c=None, bias=None, alpha=0.125, beta=0.0, ws=False, layout=RRR):
    # ws: pass the optional workspace (pre-pass operand sums, RRR only),
    # filled with garbage first -- its contents must not matter.
    m, k = a.shape
    n = b.shape[1] if layout == RRR else b.shape[0]
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, layout=layout, epilogue=epi,
                                                    bias_element=bias_kind, element=P.ElementKind.U8,
                                                    output=P.ElementKind.U8))
    work = None
    if ws and plan.workspace_size() > 0:
        work = torch.full((plan.workspace_size(),), 0xAB, dtype=torch.uint8, device="cuda:0")
    d = torch.full((m, n), 99, dtype=torch.uint8, device="cuda:0")
    plan.run(dev(a), dev(b), d, c=None if c is None else dev(c), alpha=alpha, beta=beta,
             bias=None if bias is None else dev(bias), workspace=work)
    sync()
    return d.cpu().numpy()


# (layout, ws): the u8 workspace pre-pass exists for RRR only.
U8_PATHS = [(RRR, False), (RRR, True), (RCR, False)]
_LNAME = {RRR: "rrr", RCR: "rcr"}


def _u8_b(g_or_pattern, k, n, layout):
    """B of a u8 test: [K, N] for RRR, [N, K] for RCR."""
    return g_or_pattern.reshape(k, n) if layout == RRR else g_or_pattern.reshape(n, k)


@pytest.mark.parametrize("layout,ws", U8_PATHS)
@pytest.mark.parametrize("bias_kind", [P.ElementKind.F32, P.ElementKind.I32])
@pytest.mark.parametrize("epi", EPIS)
@pytest.mark.parametrize("shape", REF_SHAPES + [(256, 256, 128), (512, 512, 256)])
def test_u8_reference_smoke_pattern(gpu, shape, epi, bias_kind, layout, ws):
    if epi == P.EpilogueKind.Identity and bias_kind == P.ElementKind.I32:
        pytest.skip("Identity has no bias")
    m, n, k = shape
    print(f"case: u8 {_LNAME[layout]} {epi.value} {bias_kind.value} {shape} ws={ws}", flush=True)
    a = ((np.arange(m * k) * 7) % 16).astype(np.uint8).reshape(m, k)
    b = _u8_b(((np.arange(k * n) * 11) % 14).astype(np.uint8), k, n, layout)
    bias = _bias(n, bias_kind)
    got = _run_u8(epi, bias_kind, a, b, bias=bias, ws=ws, layout=layout)
    want = O.gemm_u8_epi(a, b, _LNAME[layout], 0.125, 0.0, None,
                         None if epi == P.EpilogueKind.Identity else bias, ACT[epi])
    _check(got, want, epi)


@pytest.mark.parametrize("layout,ws", U8_PATHS)
@pytest.mark.parametrize("epi", EPIS)
@pytest.mark.parametrize("shape", [(256, 256, 128), (512, 768, 384), (300, 520, 200), (130, 260, 1000)])
def test_u8_full_range_with_c(gpu, shape, epi, layout, ws):
    # Full-range bytes (the flipped sign bit matters) on the DMA and the
    # general path, including a K tail (200, 1000) whose zero padding the
    # correction accounts for.
    m, n, k = shape
    print(f"case: u8 {_LNAME[layout]} random {epi.value} {shape} ws={ws}", flush=True)
    g = rng(m * 3 + n + k)
    a = g.integers(0, 256, (m, k), dtype=np.uint8)
    b = _u8_b(g.integers(0, 256, k * n, dtype=np.uint8), k, n, layout)
    c = g.integers(0, 256, (m, n), dtype=np.uint8)
    bias = (g.standard_normal(n) * 30).astype(np.float32)
    alpha = 1.0 / (64.0 * k)
    got = _run_u8(epi, P.ElementKind.F32, a, b, c=c, bias=bias, alpha=alpha, beta=0.5, ws=ws, layout=layout)
    want = O.gemm_u8_epi(a, b, _LNAME[layout], alpha, 0.5, c,
                         None if epi == P.EpilogueKind.Identity else bias, ACT[epi])
    _check(got, want, epi)


@pytest.mark.parametrize("layout,ws", U8_PATHS)
def test_u8_large_k_exact_accumulator(gpu, layout, ws):
    # alpha = 1 / 2^k-scale keeps the u8 output informative at K = 8192
    # (acc up to 255^2 * 8192 ~ 5.3e8 < 2^31): checks the 16384*K term.
    m, n, k = 256, 256, 8192
    g = rng(99)
    a = g.integers(0, 256, (m, k), dtype=np.uint8)
    b = _u8_b(g.integers(0, 256, k * n, dtype=np.uint8), k, n, layout)
    alpha = 255.0 / (255.0 * 255.0 * k)
    got = _run_u8(P.EpilogueKind.Identity, P.ElementKind.F32, a, b, alpha=alpha, ws=ws, layout=layout)
    want = O.gemm_u8_epi(a, b, _LNAME[layout], alpha)
    assert np.array_equal(got, want)


def test_u8_rcr_strided_unaligned_and_full_result(gpu):
    # RCR u8 on padded leading dimensions with a B base offset by 1 byte (the
    # general kernel's byte-granular path), BiasRelu with an i32 bias; then
    # a 1024 x 1024 x 2048 Identity result checked in full against torch's
    # int64 matmul (alpha 1/2^20 keeps the u8 output informative).
    m, n, k = 130, 260, 96
    g = rng(15)
    a_full = g.integers(0, 256, (m, k + 16), dtype=np.uint8)
    b_full = g.integers(0, 256, (n, k + 9), dtype=np.uint8)
    a_t, b_t = dev(a_full)[:, :k], dev(b_full)[:, 1:k + 1]
    d_full = torch.zeros((m, n + 4), dtype=torch.uint8, device="cuda:0")
    d = d_full[:, :n]
    bias = _bias(n, P.ElementKind.I32)
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, layout=RCR, epilogue=P.EpilogueKind.BiasRelu,
                                                    bias_element=P.ElementKind.I32, element=P.ElementKind.U8,
                                                    output=P.ElementKind.U8))
    plan.run(a_t, b_t, d, alpha=1.0 / 2048, bias=dev(bias))
    sync()
    want = O.gemm_u8_epi(a_full[:, :k], b_full[:, 1:k + 1], "rcr", 1.0 / 2048, bias=bias, act="relu")
    assert np.array_equal(d.cpu().numpy(), want)
    assert np.all(d_full[:, n:].cpu().numpy() == 0)   # padding untouched
    m = n = 1024
    k = 2048
    a = g.integers(0, 256, (m, k), dtype=np.uint8)
    b = g.integers(0, 256, (n, k), dtype=np.uint8)
    got = _run_u8(P.EpilogueKind.Identity, P.ElementKind.F32, a, b, alpha=1.0 / (1 << 20), layout=RCR)
    acc = (torch.from_numpy(a).to(torch.int64) @ torch.from_numpy(b).to(torch.int64).T).numpy()
    want = np.clip(np.rint(np.float32(1.0 / (1 << 20)) * acc.astype(np.float32)), 0, 255).astype(np.uint8)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("epi", EPIS)
def test_u8_workspace_path_bit_identical(gpu, epi):
    # The pre-pass sums and the in-loop sums are both exact: same bytes out.
    m, n, k = 512, 768, 1024
    g = rng(4242)
    a = g.integers(0, 256, (m, k), dtype=np.uint8)
    b = g.integers(0, 256, (k, n), dtype=np.uint8)
    c = g.integers(0, 256, (m, n), dtype=np.uint8)
    bias = (g.standard_normal(n) * 30).astype(np.float32)
    kw = dict(c=c, bias=bias, alpha=1.0 / (64.0 * k), beta=0.5)
    assert np.array_equal(_run_u8(epi, P.ElementKind.F32, a, b, ws=True, **kw),
                          _run_u8(epi, P.ElementKind.F32, a, b, ws=False, **kw))


@pytest.mark.parametrize("layout", [P.LayoutSku.Rcr, P.LayoutSku.Rrr])
def test_s8_saturation_of_non_finite_and_huge_bias(gpu, layout):
    # z = alpha*acc + bias with bias in {+inf, -inf, NaN, +1e10, -1e10, 0.4}:
    # the int8 store saturates to 127 / -128, NaN stores 0 (the hardware
    # conversion; the reference's sat_cast has no NaN case), finite values
    # round half to even.  Staged (whole tile) and per-quad (edge) paths.
    for m, n, k in [(256, 256, 128), (70, 36, 64)]:
        g = rng(m + n)
        a = int8_uniform(g, (m, k))
        b = int8_uniform(g, (k, n)) if layout == P.LayoutSku.Rrr else int8_uniform(g, (n, k))
        special = np.array([np.inf, -np.inf, np.nan, 1e10, -1e10, 0.4], np.float32)
        bias = special[np.arange(n) % 6]
        got = _run(layout, P.EpilogueKind.Bias, P.ElementKind.F32, a, b, bias=bias, alpha=1e-9)
        want_col = np.array([127, -128, 0, 127, -128, 0], np.int8)[np.arange(n) % 6]
        assert np.array_equal(got, np.broadcast_to(want_col, (m, n))), (m, n, k)


@pytest.mark.parametrize("elem", [P.ElementKind.S8, P.ElementKind.U8])
@pytest.mark.parametrize("epi", [P.EpilogueKind.Identity, P.EpilogueKind.BiasRelu])
@pytest.mark.parametrize("layout", [RCR, RRR])
@pytest.mark.parametrize("shape", [(512, 512, 256), (300, 520, 200), (1, 256, 4096), (4097, 256, 256)])
def test_null_c_with_beta(gpu, shape, layout, epi, elem):
    # C = NULL with beta != 0.  RCR follows the CUTLASS contract of the
    # reference (gemm_s8_rcr_sm80.cu:87-89, gemm_u8_rcr_sm80.cu:77-79): the
    # source operand is D itself, so the GEMM accumulates into D in place.
    # RRR follows its bespoke kernel (baracuda_int8_rrr_sm80.cuh:274): no
    # beta term.  Shapes reach the whole-tile DMA kernel, the general kernel
    # (K tail), the last-rows pass (M = 1) and tiles plus last rows (4097).
    m, n, k = shape
    u8 = elem == P.ElementKind.U8
    print(f"case: null C {layout.value} {epi.value} {elem.value} {shape}", flush=True)
    g = rng(m + 3 * n + 5 * k + (7 if u8 else 0))
    if u8:
        a = g.integers(0, 256, (m, k), dtype=np.uint8)
        b = _u8_b(g.integers(0, 256, k * n, dtype=np.uint8), k, n, layout)
        d0 = g.integers(0, 256, (m, n), dtype=np.uint8)
        alpha = 1.0 / (64.0 * k)
    else:
        a = int8_uniform(g, (m, k))
        b = int8_uniform(g, (k, n)) if layout == RRR else int8_uniform(g, (n, k))
        d0 = int8_uniform(g, (m, n))
        alpha = 1.0 / (16.0 * np.sqrt(k))
    bias = (g.standard_normal(n) * 8).astype(np.float32)
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, layout=layout, epilogue=epi,
                                                    bias_element=P.ElementKind.F32, element=elem, output=elem))
    d = dev(d0)
    plan.run(dev(a), dev(b), d, c=None, alpha=alpha, beta=0.5,
             bias=None if epi == P.EpilogueKind.Identity else dev(bias))
    sync()
    f = O.gemm_u8_epi if u8 else O.gemm_s8_epi
    want = f(a, b, _LNAME[layout], alpha, 0.5, d0 if layout == RCR else None,
             None if epi == P.EpilogueKind.Identity else bias, ACT[epi])
    _check(d.cpu().numpy(), want, epi)


# u8 last rows (decode-sized M, and M % 256 <= 128 under whole tile rows):
# the staged last-rows kernel with flipped operands and the correction
# folded into its accumulator.  2 / 4 / 8 row fragments, 16 / 32 / 64
# columns per workgroup, main 256x256 tiles above the rows.
U8_ROWS_SHAPES = [(1, 4096, 4096), (5, 256, 512), (33, 512, 1024), (100, 6144, 512), (128, 12288, 512),
                  (1025, 16384, 512), (1100, 16384, 1024), (20, 272, 512), (1, 256, 1024),
                  # row blocks below N = 6144: two 64-row blocks, three 32-row blocks
                  (100, 4096, 512), (90, 1024, 1024),
                  # one fragment (up to 16 rows) at 32 / 64 columns
                  (12, 14336, 1024), (9, 8192, 512)]


@pytest.mark.parametrize("layout", [RCR, RRR])
@pytest.mark.parametrize("epi", [P.EpilogueKind.Identity, P.EpilogueKind.BiasGelu, P.EpilogueKind.BiasRelu])
@pytest.mark.parametrize("shape", U8_ROWS_SHAPES)
def test_u8_last_rows(gpu, shape, epi, layout):
    # RCR: 16 / 32 / 64 columns per workgroup by N; RRR (row-major B,
    # transposing LDS reads): 64 columns where N % 64 == 0
    m, n, k = shape
    print(f"case: u8 {_LNAME[layout]} rows {epi.value} {shape}", flush=True)
    g = rng(m + 3 * n + k)
    a = g.integers(0, 256, (m, k), dtype=np.uint8)
    b = _u8_b(g.integers(0, 256, n * k, dtype=np.uint8), k, n, layout)
    c = g.integers(0, 256, (m, n), dtype=np.uint8)
    bias = (g.standard_normal(n) * 30).astype(np.float32)
    alpha = 1.0 / (64.0 * k)
    has_bias = epi != P.EpilogueKind.Identity
    got = _run_u8(epi, P.ElementKind.F32, a, b, c=c, bias=bias if has_bias else None, alpha=alpha, beta=0.5,
                  layout=layout)
    rows = slice(max(0, m - m % 256 - 2), m) if m > 256 else slice(0, m)
    want = O.gemm_u8_epi(a[rows], b, _LNAME[layout], alpha, 0.5, c[rows], bias if has_bias else None, ACT[epi])
    _check(got[rows], want, epi)


@pytest.mark.parametrize("layout", [RCR, RRR])
def test_u8_last_rows_large_k_exact(gpu, layout):
    # K = 8192 (255^2 K < 2^31): the folded 128 (sum a' + sum b') and the
    # 16384 K term, checked through an informative u8 output
    m, n, k = 16, 512, 8192
    g = rng(77)
    a = g.integers(0, 256, (m, k), dtype=np.uint8)
    b = _u8_b(g.integers(0, 256, n * k, dtype=np.uint8), k, n, layout)
    alpha = 255.0 / (255.0 * 255.0 * k)
    got = _run_u8(P.EpilogueKind.Identity, P.ElementKind.F32, a, b, alpha=alpha, layout=layout)
    assert np.array_equal(got, O.gemm_u8_epi(a, b, _LNAME[layout], alpha))


# s8 RRR last rows (decode-sized M, and M % 256 <= 128 under whole tile
# rows): the staged last-rows kernel reading row-major B with transposing
# LDS reads; 16 / 32 / 64 columns per workgroup by the last-rows rule (N
# below 6144 / from 6144 / from 12288), 2 / 4 / 8 row fragments, main RRR
# tiles above the rows.
RRR_ROWS_SHAPES = [(1, 4096, 4096), (5, 256, 512), (33, 512, 1024), (20, 288, 512), (100, 272, 512),
                   (128, 1024, 2048), (1025, 16384, 512), (1100, 16384, 1024), (20, 6144, 512), (100, 4096, 512),
                   (9, 8192, 512), (16, 14336, 512)]


@pytest.mark.parametrize("epi", [P.EpilogueKind.Identity, P.EpilogueKind.BiasGelu, P.EpilogueKind.BiasRelu])
@pytest.mark.parametrize("shape", RRR_ROWS_SHAPES)
def test_s8_rrr_last_rows(gpu, shape, epi):
    m, n, k = shape
    print(f"case: s8 rrr rows {epi.value} {shape}", flush=True)
    g = rng(m + 5 * n + k)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (k, n))
    c = int8_uniform(g, (m, n))
    bias = (g.standard_normal(n) * 20).astype(np.float32)
    has_bias = epi != P.EpilogueKind.Identity
    alpha = 1.0 / (16.0 * k)
    got = _run(RRR, epi, P.ElementKind.F32, a, b, c=c, bias=bias if has_bias else None, alpha=alpha, beta=0.5)
    rows = slice(max(0, m - m % 256 - 2), m) if m > 256 else slice(0, m)
    want = O.gemm_s8_epi(a[rows], b, "rrr", alpha, 0.5, c[rows], bias if has_bias else None, ACT[epi])
    _check(got[rows], want, epi)


@pytest.mark.parametrize("layout,shape", [(RCR, (200, 512, 1024)), (RCR, (384, 256, 512)), (RCR, (512, 512, 512)),
                                          (RRR, (200, 512, 1024)), (RRR, (256, 512, 512)), (RRR, (384, 256, 512)),
                                          (RCR, (512, 4096, 512)), (RRR, (300, 4096, 512))])
def test_u8_small_grid_row_blocks(gpu, layout, shape):
    # u8 grids of at most 512 rows (RRR: 256, or 512 off the 256 grid): every row as 64-row
    # blocks of the last-rows kernel (128-row blocks where the 64-row ones would
    # need a second round: 512 x 4096, 300 x 4096); the whole output against the oracle
    m, n, k = shape
    print(f"case: u8 {_LNAME[layout]} row blocks {shape}", flush=True)
    g = rng(m + 11 * n + k)
    a = g.integers(0, 256, (m, k), dtype=np.uint8)
    b = _u8_b(g.integers(0, 256, n * k, dtype=np.uint8), k, n, layout)
    c = g.integers(0, 256, (m, n), dtype=np.uint8)
    bias = (g.standard_normal(n) * 30).astype(np.float32)
    alpha = 1.0 / (64.0 * k)
    got = _run_u8(P.EpilogueKind.BiasRelu, P.ElementKind.F32, a, b, c=c, bias=bias, alpha=alpha, beta=0.5,
                  layout=layout)
    want = O.gemm_u8_epi(a, b, _LNAME[layout], alpha, 0.5, c, bias, "relu")
    assert np.array_equal(got, want)


@pytest.mark.parametrize("shape", [(200, 512, 1024), (512, 256, 512), (300, 288, 512), (300, 4096, 512)])
def test_s8_rrr_small_grid_row_blocks(gpu, shape):
    # s8 RRR grids of at most 512 rows: every row as 128-row blocks of the
    # last-rows kernel (row-major B); the whole output against the oracle
    m, n, k = shape
    print(f"case: s8 rrr row blocks {shape}", flush=True)
    g = rng(m + 13 * n + k)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (k, n))
    c = int8_uniform(g, (m, n))
    bias = (g.standard_normal(n) * 20).astype(np.float32)
    alpha = 1.0 / (16.0 * k)
    got = _run(RRR, P.EpilogueKind.BiasRelu, P.ElementKind.F32, a, b, c=c, bias=bias, alpha=alpha, beta=0.5)
    assert np.array_equal(got, O.gemm_s8_epi(a, b, "rrr", alpha, 0.5, c, bias, "relu"))
