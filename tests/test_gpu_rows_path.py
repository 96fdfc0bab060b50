"""GPU parity of the int8 RCR last-rows path: M % 256 in [1, 64] (M > 256,
N % 16 == 0, K % 128 == 0) runs whole 256-row tiles plus a streamed pass
over the last rows.  Every SKU family of the RCR launch goes through it;
all outputs bit-exact against the oracle (int64 matmul for int32 out)."""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from baracuda_amd.ffi import lib
from oracle import oracle as O
from oracle.inputs import int8_uniform, rng
from tests.gpu_util import dev, host_bits16, sync

pytestmark = pytest.mark.gpu

# (M, N, K): 1 / 12 / 16 last rows (one 16-row fragment), 25 / 32 (two),
# 44 / 64 (four); N with and without a partial 256-column tile; K of 6 / 10 /
# 18 / 64 / 128 chunks of 64 bytes (each wave's batches, their remainder, or
# both).
SHAPES = [(257, 256, 384), (268, 272, 640), (272, 512, 4096), (528, 1040, 1152), (769, 256, 8192),
          (281, 256, 640), (544, 272, 4096), (300, 1040, 1152), (320, 512, 8192)]


@pytest.mark.parametrize("shape", SHAPES)
def test_rows_path_i32_s8_w8a8(gpu, shape):
    m, n, k = shape
    print(f"case: rows path {shape}", flush=True)
    g = rng(m * 7 + n + k)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    d = torch.full((m, n), -7, dtype=torch.int32, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.I32)).run(dev(a), dev(b), d)
    sync()
    assert np.array_equal(d.cpu().numpy(), a.astype(np.int64) @ b.astype(np.int64).T)

    c = int8_uniform(g, (m, n))
    d8 = torch.full((m, n), 99, dtype=torch.int8, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k)).run(dev(a), dev(b), d8, c=dev(c), alpha=0.003, beta=0.5)
    sync()
    assert np.array_equal(d8.cpu().numpy(), O.gemm_s8_rcr_s8(a, b, 0.003, 0.5, c))

    sa = g.uniform(0.005, 0.02, m).astype(np.float32)
    sw = g.uniform(0.001, 0.01, n).astype(np.float32)
    dw = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16)).run(
        dev(a), dev(b), dw, scale_a=dev(sa), scale_b=dev(sw))
    sync()
    assert np.array_equal(host_bits16(dw), O.gemm_w8a8_bf16(a, b, sa, sw, nthreads=8))


@pytest.mark.parametrize("shape", SHAPES[:3])
def test_rows_path_bias_gelu(gpu, shape):
    m, n, k = shape
    print(f"case: rows path bias_gelu {shape}", flush=True)
    g = rng(m + 3 * n + k)
    a, b, c = int8_uniform(g, (m, k)), int8_uniform(g, (n, k)), int8_uniform(g, (m, n))
    bias = (g.standard_normal(n) * 6).astype(np.float32)
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, epilogue=P.EpilogueKind.BiasGelu,
                                                    bias_element=P.ElementKind.F32))
    d = torch.full((m, n), 99, dtype=torch.int8, device="cuda:0")
    plan.run(dev(a), dev(b), d, c=dev(c), alpha=0.004, beta=0.25, bias=dev(bias))
    sync()
    assert np.array_equal(d.cpu().numpy(), O.gemm_s8_epi(a, b, "rcr", 0.004, 0.25, c, bias, "gelu"))


@pytest.mark.parametrize("shape", SHAPES[1:4])
def test_rows_path_quantized_linear_f32_f64(gpu, shape):
    # f32: y = (sa*sw)*acc in f32; f64: f64 scales narrowed to f32, the same
    # product, widened (compose.cu:27-28).
    m, n, k = shape
    print(f"case: rows path quantized_linear {shape}", flush=True)
    g = rng(m + n + 5 * k)
    a, w = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    acc = O.gemm_s8_rcr_i32(a, w).astype(np.float32)
    stream = torch.cuda.current_stream().cuda_stream
    sa = g.uniform(0.005, 0.02, m).astype(np.float32)
    sw = g.uniform(0.001, 0.01, n).astype(np.float32)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    tw, ta, tsa, tsw = dev(w), dev(a), dev(sa), dev(sw)
    assert lib().quantized_linear_w8a8_f32_gfx950_run(m, n, k, tw.data_ptr(), ta.data_ptr(), tsa.data_ptr(),
                                                      tsw.data_ptr(), out.data_ptr(), None, 0, stream) == 0
    sync()
    assert np.array_equal(out.cpu().numpy(), (sa[:, None] * sw[None, :]).astype(np.float32) * acc)
    sa64, sw64 = g.uniform(0.005, 0.02, m), g.uniform(0.001, 0.01, n)
    out64 = torch.empty((m, n), dtype=torch.float64, device="cuda:0")
    tsa64, tsw64 = dev(sa64), dev(sw64)
    assert lib().quantized_linear_w8a8_f64_gfx950_run(m, n, k, tw.data_ptr(), ta.data_ptr(), tsa64.data_ptr(),
                                                      tsw64.data_ptr(), out64.data_ptr(), None, 0, stream) == 0
    sync()
    want64 = ((sa64.astype(np.float32)[:, None] * sw64.astype(np.float32)[None, :]).astype(np.float32)
              * acc).astype(np.float64)
    assert np.array_equal(out64.cpu().numpy(), want64)


def test_rows_path_takes_no_workspace(gpu):
    # M = 4097: the tail split's workspace is no longer asked for
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(4097, 4096, 4096, output=P.ElementKind.Bf16))
    assert plan.workspace_size() == 0
