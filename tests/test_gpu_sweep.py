"""Seeded random-shape sweep over the GEMM SKUs (GPU parity).

Each case draws (M, N, K) — K a multiple of 128 (LDS-DMA path, edge tiles)
or any K (general kernel) — and checks, with and without the optional
workspace where the plan reports one:
  * int8 RCR int32 out: bit-exact against an int64 matmul (numpy);
  * int8 RCR s8 out with C and beta: bit-exact against the oracle;
  * W8A8 bf16 out: bit-exact against the oracle's f32 epilogue;
  * u8 RCR u8 out: bit-exact against the oracle;
  * FP8 e4m3 RCR f32 out: within 1e-3 relative of the exact f64 sum, with the
    FP8_FLOOR * sum|a*b| floor of the other FP8 tests;
  * FP8 fp8-out (e4m3 RRR, e5m2 RCR / RRR) with C and BiasRelu: one grid step;
  * RRR s8 BiasRelu with C and u8 RRR (with / without workspace): bit-exact.
"""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from oracle import oracle as O
from oracle.inputs import int8_uniform, rng
from tests.gpu_util import FP8_FLOOR, dev, host_bits16, sync

pytestmark = pytest.mark.gpu


def _shapes(count, seed):
    g = rng(seed)
    out = []
    for i in range(count):
        m, n = int(g.integers(1, 700)), int(g.integers(1, 700))
        k = int(g.integers(1, 13)) * 128 if i % 3 else int(g.integers(1, 1500))
        out.append((m, n, k))
    return out


SHAPES = _shapes(24, 2024)


def _ws(plan, use):
    n = plan.workspace_size()
    if not use or n == 0:
        return None
    return torch.full((n,), 0x5A, dtype=torch.uint8, device="cuda:0")   # contents must not matter


@pytest.mark.parametrize("use_ws", [False, True])
@pytest.mark.parametrize("shape", SHAPES)
def test_int8_sweep(gpu, shape, use_ws):
    m, n, k = shape
    print(f"case: sweep int8 {shape} ws={use_ws}", flush=True)
    g = rng(m * 1009 + n * 31 + k)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    pi = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.I32))
    d = torch.full((m, n), -7, dtype=torch.int32, device="cuda:0")
    pi.run(dev(a), dev(b), d, workspace=_ws(pi, use_ws))
    sync()
    assert np.array_equal(d.cpu().numpy(), a.astype(np.int64) @ b.astype(np.int64).T)

    c = int8_uniform(g, (m, n))
    ps = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k))
    d8 = torch.full((m, n), 99, dtype=torch.int8, device="cuda:0")
    ps.run(dev(a), dev(b), d8, c=dev(c), alpha=0.003, beta=0.5, workspace=_ws(ps, use_ws))
    sync()
    assert np.array_equal(d8.cpu().numpy(), O.gemm_s8_rcr_s8(a, b, 0.003, 0.5, c))

    sa = g.uniform(0.005, 0.02, m).astype(np.float32)
    sw = g.uniform(0.001, 0.01, n).astype(np.float32)
    pw = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16))
    dw = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
    pw.run(dev(a), dev(b), dw, scale_a=dev(sa), scale_b=dev(sw), workspace=_ws(pw, use_ws))
    sync()
    assert np.array_equal(host_bits16(dw), O.gemm_w8a8_bf16(a, b, sa, sw, nthreads=8))


@pytest.mark.parametrize("shape", SHAPES[::2])
def test_u8_rcr_sweep(gpu, shape):
    m, n, k = shape
    print(f"case: sweep u8 rcr {shape}", flush=True)
    g = rng(m + 7 * n + 13 * k)
    a = g.integers(0, 256, (m, k)).astype(np.uint8)
    b = g.integers(0, 256, (n, k)).astype(np.uint8)
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, layout=P.LayoutSku.Rcr, element=P.ElementKind.U8,
                                                    output=P.ElementKind.U8))
    d = torch.full((m, n), 99, dtype=torch.uint8, device="cuda:0")
    alpha = 1.0 / (128.0 * k)
    plan.run(dev(a), dev(b), d, alpha=alpha)
    sync()
    assert np.array_equal(d.cpu().numpy(), O.gemm_u8_epi(a, b, "rcr", alpha))


@pytest.mark.parametrize("shape", SHAPES[1::2])
def test_fp8_sweep(gpu, shape):
    m, n, k = shape
    print(f"case: sweep fp8 {shape}", flush=True)
    g = rng(m + 3 * n + 5 * k)
    xa = g.standard_normal((m, k)).astype(np.float32)
    xb = g.standard_normal((n, k)).astype(np.float32)
    a = torch.from_numpy(xa / (np.abs(xa).max() / 448.0)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    b = torch.from_numpy(xb / (np.abs(xb).max() / 448.0)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    d = torch.zeros((m, n), dtype=torch.float32, device="cuda:0")
    P.Fp8GemmPlan.select(P.Fp8GemmDescriptor(m, n, k, output=P.ElementKind.F32)).run(dev(a), dev(b), d, alpha=1.0)
    sync()
    exact = O.gemm_fp8_e4m3_f64(a, b, nthreads=8)
    ta, tb = np.abs(O.e4m3_to_f32(a).astype(np.float64)), np.abs(O.e4m3_to_f32(b).astype(np.float64))
    err = np.abs(d.cpu().numpy().astype(np.float64) - exact)
    assert np.all(err <= 1e-3 * np.abs(exact) + FP8_FLOOR * (ta @ tb.T)), err.max()


@pytest.mark.parametrize("shape", SHAPES)
def test_int8_rrr_bias_relu_sweep(gpu, shape):
    # RRR (B [K, N] row-major) s8 out, BiasRelu with an f32 bias and C:
    # bit-exact against the oracle.
    m, n, k = shape
    print(f"case: sweep rrr bias_relu {shape}", flush=True)
    g = rng(3 * m + n + 17 * k)
    a, b, c = int8_uniform(g, (m, k)), int8_uniform(g, (k, n)), int8_uniform(g, (m, n))
    bias = (g.standard_normal(n) * 6).astype(np.float32)
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, layout=P.LayoutSku.Rrr,
                                                    epilogue=P.EpilogueKind.BiasRelu,
                                                    bias_element=P.ElementKind.F32))
    d = torch.full((m, n), 99, dtype=torch.int8, device="cuda:0")
    plan.run(dev(a), dev(b), d, c=dev(c), alpha=0.004, beta=0.25, bias=dev(bias))
    sync()
    assert np.array_equal(d.cpu().numpy(), O.gemm_s8_epi(a, b, "rrr", 0.004, 0.25, c, bias, "relu"))


@pytest.mark.parametrize("use_ws", [False, True])
@pytest.mark.parametrize("shape", SHAPES[::3])
def test_u8_rrr_sweep(gpu, shape, use_ws):
    m, n, k = shape
    print(f"case: sweep u8 rrr {shape} ws={use_ws}", flush=True)
    g = rng(m + 11 * n + 5 * k)
    a = g.integers(0, 256, (m, k)).astype(np.uint8)
    b = g.integers(0, 256, (k, n)).astype(np.uint8)
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, layout=P.LayoutSku.Rrr, element=P.ElementKind.U8,
                                                    output=P.ElementKind.U8))
    d = torch.full((m, n), 99, dtype=torch.uint8, device="cuda:0")
    alpha = 1.0 / (128.0 * k)
    plan.run(dev(a), dev(b), d, alpha=alpha, workspace=_ws(plan, use_ws))
    sync()
    assert np.array_equal(d.cpu().numpy(), O.gemm_u8_epi(a, b, "rrr", alpha))


@pytest.mark.parametrize("shape", SHAPES[2::3])
@pytest.mark.parametrize("fmt,layout", [("e4m3", P.LayoutSku.Rrr), ("e5m2", P.LayoutSku.Rcr),
                                        ("e5m2", P.LayoutSku.Rrr)])
def test_fp8_out_with_c_sweep(gpu, shape, fmt, layout):
    # fp8-out SKUs with C (beta = 0.5) and BiasRelu: within one grid step of
    # the exactly rounded result plus the MFMA summation floor, differences
    # on under 2% of the outputs (the bar of test_gpu_fp8_epi).
    from tests.test_gpu_fp8_epi import _run as f8_run, _steps, _want as f8_want
    m, n, k = shape
    print(f"case: sweep fp8 out {fmt} {layout.value} {shape}", flush=True)
    g = rng(7 * m + n + k)
    a = O.f32_to_fp8(g.standard_normal((m, k)).astype(np.float32), fmt)
    b = O.f32_to_fp8(g.standard_normal((k, n) if layout == P.LayoutSku.Rrr else (n, k)).astype(np.float32), fmt)
    c = O.f32_to_fp8(g.standard_normal((m, n)).astype(np.float32), fmt)
    bias = g.standard_normal(n).astype(np.float32)
    alpha = 1.0 / 16
    epi = P.EpilogueKind.BiasRelu
    got = f8_run(fmt, layout, epi, a, b, c=c, bias=bias, alpha=alpha, beta=0.5)
    want = f8_want(fmt, layout, epi, a, b, c, bias, alpha, 0.5)
    fa = np.abs(O.fp8_to_f32(a, fmt).astype(np.float64))
    fb = np.abs(O.fp8_to_f32(b, fmt).astype(np.float64))
    floor = FP8_FLOOR * alpha * (fa @ (fb if layout == P.LayoutSku.Rrr else fb.T))
    st = _steps(got, want, fmt, floor)
    assert st.max() <= 1.0 and (got != want).mean() < 0.02


def _small_m_shapes(count, seed):
    # the W8A8 last-rows kernels: M <= 128 (no tiles) with N % 16 == 0 and
    # K % 128 == 0; K % 1024 == 0 and M <= 32 take the LDS-streamed B kernel
    g = rng(seed)
    out = []
    for i in range(count):
        m = int(g.integers(1, 33)) if i % 2 == 0 else int(g.integers(1, 129))
        n = 16 * int(g.integers(1, 160))
        k = 1024 * int(g.integers(1, 9)) if i % 4 != 3 else 128 * int(g.integers(1, 40))
        out.append((m, n, k))
    return out


@pytest.mark.parametrize("shape", _small_m_shapes(16, 77))
def test_int8_small_m_sweep(gpu, shape):
    m, n, k = shape
    print(f"case: sweep small-M int8 {shape}", flush=True)
    g = rng(m * 7 + n * 13 + k)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    pi = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.I32))
    d = torch.full((m, n), -7, dtype=torch.int32, device="cuda:0")
    pi.run(dev(a), dev(b), d)
    sync()
    assert np.array_equal(d.cpu().numpy(), a.astype(np.int64) @ b.astype(np.int64).T)
    sa = g.uniform(0.005, 0.02, m).astype(np.float32)
    sw = g.uniform(0.001, 0.01, n).astype(np.float32)
    dw = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16)).run(
        dev(a), dev(b), dw, scale_a=dev(sa), scale_b=dev(sw))
    sync()
    assert np.array_equal(host_bits16(dw), O.gemm_w8a8_bf16(a, b, sa, sw, nthreads=8))
