"""hipGraph capture of the W8A8 pipeline: per-token int8 quantization of bf16
activations followed by the W8A8 GEMM (the reference's QuantizedLinearPlan
two-pass flow) recorded once and replayed.  Neither kernel allocates, sets
memory or synchronizes, so the captured graph holds only the two kernels.
Every replay gets new activations, runs eager work in between, and must match
the eager result bit for bit.
"""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from tests.gpu_util import sync

pytestmark = pytest.mark.gpu


def _pipeline(x, q, sa, w, sw, out, stream=None):
    P.dynamic_range_quantize_per_token_sym(x, sa, q, stream=stream)
    m, k = x.shape
    n = w.shape[0]
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16)).run(
        q, w, out, scale_a=sa, scale_b=sw, stream=stream)


@pytest.mark.parametrize("shape", [(256, 512, 1024), (200, 384, 520)])   # DMA path, general path
def test_quantize_w8a8_graph_replays_match_eager(gpu, shape):
    m, n, k = shape
    torch.manual_seed(m + n + k)
    dev = "cuda:0"
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev)
    sw = torch.rand(n, device=dev) * 0.009 + 0.001
    x = torch.randn((m, k), device=dev).to(torch.bfloat16)
    q = torch.empty((m, k), dtype=torch.int8, device=dev)
    sa = torch.empty(m, dtype=torch.float32, device=dev)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    # warm the plans (and any lazy library state) outside the capture
    _pipeline(x, q, sa, w, sw, out)
    sync()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _pipeline(x, q, sa, w, sw, out)
    for rep in range(4):
        x.copy_(torch.randn((m, k), device=dev).to(torch.bfloat16) * (rep + 1))
        q_e = torch.empty_like(q)
        sa_e = torch.empty_like(sa)
        out_e = torch.empty_like(out)
        _pipeline(x, q_e, sa_e, w, sw, out_e)          # eager reference
        sync()
        g.replay()
        sync()
        print(f"case: graph replay {rep} {shape}", flush=True)
        assert torch.equal(q, q_e) and torch.equal(sa, sa_e)
        assert torch.equal(out.view(torch.int16), out_e.view(torch.int16))
        _ = (torch.randn(1024, device=dev) @ torch.randn(1024, device=dev))   # eager work in between
