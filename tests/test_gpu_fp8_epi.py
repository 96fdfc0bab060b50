"""GPU parity of the FP8 fp8-out SKUs -- {e4m3, e5m2} x {RCR, RRR} x {Identity,
Bias, BiasRelu, BiasGelu, BiasSilu} -- against the CPU oracle.

Inputs of the reference smoke tests (crates/baracuda-kernels/tests/
fp8_bias_smoke.rs, fp8_e5m2_rrr_smoke.rs): a = ((5i)%13-6)/8, b = ((7i)%11-5)/8
quantized to the encoding, alpha = 0.25, bias ((j%5)-2)/2.  Every product and
partial sum of these is exact in f32, so Identity / Bias / BiasRelu are
bit-exact; BiasGelu / BiasSilu are within one grid step (the reference allows
two).  Random N(0,1) operands with C, on the LDS-DMA shapes too: within one
grid step plus the f8f6f4 MFMA's own summation error (FP8_FLOOR * alpha * sum|a*b|,
the floor the e4m3 accumulator tests establish against hipBLASLt) of the
exactly rounded result, with differences on under 2% of the outputs.
"""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from oracle import oracle as O
from oracle.inputs import rng
from tests.gpu_util import FP8_FLOOR, dev, sync

pytestmark = pytest.mark.gpu

ENC = {"e4m3": P.ElementKind.Fp8E4M3, "e5m2": P.ElementKind.Fp8E5M2}
EPIS = [P.EpilogueKind.Identity, P.EpilogueKind.Bias, P.EpilogueKind.BiasRelu,
        P.EpilogueKind.BiasGelu, P.EpilogueKind.BiasSilu]
ACT = {P.EpilogueKind.Identity: None, P.EpilogueKind.Bias: None, P.EpilogueKind.BiasRelu: "relu",
       P.EpilogueKind.BiasGelu: "gelu", P.EpilogueKind.BiasSilu: "silu"}
# The reference smoke shapes (general path) plus two LDS-DMA shapes.
REF_SHAPES = [(64, 64, 32), (128, 128, 128), (256, 128, 64), (100, 70, 50), (256, 256, 128),
              (512, 512, 256)]
BIG_SHAPES = [(256, 256, 128), (512, 768, 384), (300, 520, 200)]


def _grid(x, fmt):
    a = np.abs(x).astype(np.float64)
    if fmt == "e4m3":
        small, lo, mb = 2.0 ** -6, 2.0 ** -9, 3
    else:
        small, lo, mb = 2.0 ** -14, 2.0 ** -16, 2
    e = np.floor(np.log2(np.where(a >= small, a, 1.0)))
    return np.where(a >= small, np.exp2(e - mb), lo)


def _run(fmt, layout, epi, a, b, c=None, bias=None, alpha=0.25, beta=0.0):
    m, k = a.shape
    n = b.shape[1] if layout == P.LayoutSku.Rrr else b.shape[0]
    plan = P.Fp8GemmPlan.select(P.Fp8GemmDescriptor(m, n, k, layout=layout, epilogue=epi,
                                                    output=ENC[fmt], element=ENC[fmt]))
    d = torch.full((m, n), 0x55, dtype=torch.uint8, device="cuda:0")
    plan.run(dev(a), dev(b), d, c=None if c is None else dev(c), alpha=alpha, beta=beta,
             bias=None if bias is None else dev(bias))
    sync()
    return d.cpu().numpy()


def _want(fmt, layout, epi, a, b, c, bias, alpha, beta):
    acc = O.gemm_fp8_f64(a, b, fmt, "rrr" if layout == P.LayoutSku.Rrr else "rcr", nthreads=8)
    return O.fp8_epilogue(acc, fmt, alpha, beta, c, None if epi == P.EpilogueKind.Identity else bias,
                          ACT[epi])


def _steps(got, want, fmt, floor=0.0):
    g, w = O.fp8_to_f32(got, fmt), O.fp8_to_f32(want, fmt)
    return np.maximum(np.abs(g - w) - floor, 0.0) / _grid(np.maximum(np.abs(g), np.abs(w)), fmt)


@pytest.mark.parametrize("epi", EPIS)
@pytest.mark.parametrize("layout", [P.LayoutSku.Rcr, P.LayoutSku.Rrr])
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape", REF_SHAPES)
def test_reference_smoke_pattern(gpu, shape, fmt, layout, epi):
    m, n, k = shape
    print(f"case: fp8 {fmt} {layout.value} {epi.value} {shape}", flush=True)
    a = O.f32_to_fp8((((np.arange(m * k) * 5) % 13) - 6.0) * 0.125, fmt).reshape(m, k)
    bl = O.f32_to_fp8((((np.arange(k * n) * 7) % 11) - 5.0) * 0.125, fmt)
    b = bl.reshape(k, n) if layout == P.LayoutSku.Rrr else bl.reshape(n, k)
    bias = (((np.arange(n) % 5) - 2) * 0.5).astype(np.float32)
    got = _run(fmt, layout, epi, a, b, bias=bias)
    want = _want(fmt, layout, epi, a, b, None, bias, 0.25, 0.0)
    if ACT[epi] in (None, "relu"):
        assert np.array_equal(got, want)
    else:
        assert _steps(got, want, fmt).max() <= 1.0


@pytest.mark.parametrize("epi", EPIS)
@pytest.mark.parametrize("layout", [P.LayoutSku.Rcr, P.LayoutSku.Rrr])
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape", BIG_SHAPES)
def test_random_with_c(gpu, shape, fmt, layout, epi):
    m, n, k = shape
    print(f"case: fp8 random {fmt} {layout.value} {epi.value} {shape}", flush=True)
    g = rng(m + 5 * n + 3 * k)
    a = O.f32_to_fp8(g.standard_normal((m, k)).astype(np.float32), fmt)
    b = O.f32_to_fp8(g.standard_normal((k, n) if layout == P.LayoutSku.Rrr else (n, k)).astype(np.float32), fmt)
    c = O.f32_to_fp8(g.standard_normal((m, n)).astype(np.float32), fmt)
    bias = g.standard_normal(n).astype(np.float32)
    alpha = 1.0 / 16
    got = _run(fmt, layout, epi, a, b, c=c, bias=bias, alpha=alpha, beta=0.5)
    want = _want(fmt, layout, epi, a, b, c, bias, alpha, 0.5)
    fa = np.abs(O.fp8_to_f32(a, fmt).astype(np.float64))
    fb = np.abs(O.fp8_to_f32(b, fmt).astype(np.float64))
    absum = fa @ (fb if layout == P.LayoutSku.Rrr else fb.T)
    floor = FP8_FLOOR * alpha * absum
    st = _steps(got, want, fmt, floor)
    assert st.max() <= 1.0 and (got != want).mean() < 0.02


def test_e5m2_rrr_dma_matches_rcr_bitwise(gpu):
    # The RRR DMA path (transposing LDS reads) and the RCR DMA path see the
    # same operands in different layouts: their fp8 outputs must agree bit
    # for bit, since both run the same MFMA sequence over the same k order.
    m, n, k = 512, 512, 1024
    g = rng(31)
    a = O.f32_to_fp8(g.standard_normal((m, k)).astype(np.float32), "e5m2")
    bt = O.f32_to_fp8(g.standard_normal((n, k)).astype(np.float32), "e5m2")
    rcr = _run("e5m2", P.LayoutSku.Rcr, P.EpilogueKind.Identity, a, bt, alpha=1.0 / 32)
    rrr = _run("e5m2", P.LayoutSku.Rrr, P.EpilogueKind.Identity, a, np.ascontiguousarray(bt.T), alpha=1.0 / 32)
    assert np.array_equal(rcr, rrr)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape", [(100, 70, 50), (256, 256, 128)])
def test_saturating_outputs(gpu, fmt, shape):
    # A large alpha pushes most outputs past max finite: satfinite clamps to
    # +-max (0x7e / 0x7b), never inf or NaN; exact pattern sums keep it bit-exact.
    m, n, k = shape
    a = O.f32_to_fp8((((np.arange(m * k) * 5) % 13) - 6.0) * 0.125, fmt).reshape(m, k)
    b = O.f32_to_fp8((((np.arange(k * n) * 7) % 11) - 5.0) * 0.125, fmt).reshape(n, k)
    alpha = 4096.0 if fmt == "e4m3" else 2.0 ** 19
    got = _run(fmt, P.LayoutSku.Rcr, P.EpilogueKind.Identity, a, b, alpha=alpha)
    want = _want(fmt, P.LayoutSku.Rcr, P.EpilogueKind.Identity, a, b, None, None, alpha, 0.0)
    assert np.array_equal(got, want)
    mx = 0x7E if fmt == "e4m3" else 0x7B
    assert ((got & 0x7F) == mx).mean() > 0.3


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("shape", [(256, 256, 128), (64, 64, 32)])
def test_c_roundtrip_every_code(gpu, shape, fmt):
    # alpha = 0, beta = 1: D = enc(0 * acc + dec(C)) = C for every code but
    # 0x80 (+-0 by the sign of acc), the NaN codes (-> sign | 0x7f) and the e5m2
    # infinities (-> the max finite, satfinite): the C decode on the LDS-DMA
    # and general paths over all 256 codes, NaN signs included.
    m, n, k = shape
    print(f"case: fp8 C roundtrip {fmt} {shape}", flush=True)
    g = rng(k)
    a = O.f32_to_fp8(g.standard_normal((m, k)).astype(np.float32), fmt)
    b = O.f32_to_fp8(g.standard_normal((n, k)).astype(np.float32), fmt)
    c = (np.arange(m * n) % 256).astype(np.uint8).reshape(m, n)
    got = _run(fmt, P.LayoutSku.Rcr, P.EpilogueKind.Identity, a, b, c=c, alpha=0.0, beta=1.0)
    nan = (c & 0x7F) == 0x7F if fmt == "e4m3" else (c & 0x7F) > 0x7C
    want = np.where(nan, (c & 0x80) | 0x7F, c).astype(np.uint8)
    if fmt == "e5m2":
        want = np.where((c & 0x7F) == 0x7C, (c & 0x80) | 0x7B, want).astype(np.uint8)
    # -0 + (0 * acc): -0 where acc < 0, +0 otherwise
    zero = c == 0x80
    assert np.all((got[zero] == 0x80) | (got[zero] == 0x00))
    assert np.array_equal(got[~zero], want[~zero])
