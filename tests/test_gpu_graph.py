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


def _decode_calls(kind):
    """(inputs to refresh, call(out)) of one decode-sized path."""
    dev = "cuda:0"
    if kind == "w8a8_m1":          # one-row dot4 kernel
        m, n, k = 1, 4096, 4096
        a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=dev)
        w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev)
        sa, sw = torch.rand(m, device=dev) + 0.01, torch.rand(n, device=dev) * 0.01
        plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16))
        return a, (m, n), torch.bfloat16, lambda o: plan.run(a, w, o, scale_a=sa, scale_b=sw)
    if kind == "w8a8_m40_wide":    # staged last rows, 64 columns per workgroup
        m, n, k = 40, 14336, 1024
        a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=dev)
        w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev)
        sa, sw = torch.rand(m, device=dev) + 0.01, torch.rand(n, device=dev) * 0.01
        plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16))
        return a, (m, n), torch.bfloat16, lambda o: plan.run(a, w, o, scale_a=sa, scale_b=sw)
    if kind == "fp8_m16":          # FP8 last rows
        m, n, k = 16, 14336, 1024
        a = torch.randint(-100, 100, (m, k), dtype=torch.int8, device=dev).view(torch.uint8)
        b = torch.randint(-100, 100, (n, k), dtype=torch.int8, device=dev).view(torch.uint8)
        plan = P.Fp8GemmPlan.select(P.Fp8GemmDescriptor(m, n, k, output=P.ElementKind.Bf16))
        return a, (m, n), torch.bfloat16, lambda o: plan.run(a, b, o, scale_a=0.01, scale_b=0.02)
    if kind == "u8_rrr_m8":        # u8 RRR last rows (flip + transposing reads)
        m, n, k = 8, 1024, 2048
        a = torch.randint(0, 256, (m, k), dtype=torch.uint8, device=dev)
        b = torch.randint(0, 256, (k, n), dtype=torch.uint8, device=dev)
        plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, layout=P.LayoutSku.Rrr, element=P.ElementKind.U8,
                                                        output=P.ElementKind.U8))
        return a, (m, n), torch.uint8, lambda o: plan.run(a, b, o, alpha=1.0 / (64 * k))
    if kind == "fp8_m1":           # FP8 one-row FMA kernel
        m, n, k = 1, 4096, 2048
        a = torch.randint(-100, 100, (m, k), dtype=torch.int8, device=dev).view(torch.uint8)
        b = torch.randint(-100, 100, (n, k), dtype=torch.int8, device=dev).view(torch.uint8)
        plan = P.Fp8GemmPlan.select(P.Fp8GemmDescriptor(m, n, k, output=P.ElementKind.Bf16))
        return a, (m, n), torch.bfloat16, lambda o: plan.run(a, b, o, scale_a=0.01, scale_b=0.02)
    if kind == "w8a8_m100_blocks":  # 33-128 last rows as row blocks (blockIdx.y)
        m, n, k = 100, 4096, 1024
        a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=dev)
        w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev)
        sa, sw = torch.rand(m, device=dev) + 0.01, torch.rand(n, device=dev) * 0.01
        plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16))
        return a, (m, n), torch.bfloat16, lambda o: plan.run(a, w, o, scale_a=sa, scale_b=sw)
    # int8 MoE decode: counts and offsets in the decode kernels; 3 tokens top-2
    # (6 pairs) take the dot4 row kernel, 4 tokens the staged 16-row blocks
    from oracle.inputs import moe_routing
    tokens, E, topk, n, k = (3 if kind == "moe_decode_row" else 4), 8, 2, 2048, 1024
    sid, eid = moe_routing(tokens, E, topk, seed=3)
    x = torch.randint(-127, 128, (tokens, k), dtype=torch.int8, device=dev)
    w = torch.randint(-127, 128, (E, n, k), dtype=torch.int8, device=dev)
    sa, sw = torch.rand(tokens, device=dev) + 0.01, torch.rand(E * n, device=dev) * 0.01
    cnt = torch.empty(E, dtype=torch.int32, device=dev)
    off = torch.empty(E + 1, dtype=torch.int32, device=dev)
    dsid, deid = torch.from_numpy(sid).to(dev), torch.from_numpy(eid).to(dev)
    plan = P.MoeS8GroupedPlan.select(E, topk, tokens * topk, n, k)
    return x, (tokens * topk, n), torch.bfloat16, lambda o: plan.run(x, w, dsid, deid, o, cnt, off, sa, sw)


@pytest.mark.parametrize("kind", ["w8a8_m1", "w8a8_m40_wide", "fp8_m16", "u8_rrr_m8", "moe_decode", "fp8_m1",
                                  "w8a8_m100_blocks", "moe_decode_row"])
def test_decode_paths_graph_replays_match_eager(gpu, kind):
    # The decode-sized passes allocate nothing and set no memory: captured
    # once, every replay (new inputs, eager work in between) equals the eager
    # call bit for bit.
    a, oshape, odt, call = _decode_calls(kind)
    dev = "cuda:0"
    out = torch.zeros(oshape, dtype=odt, device=dev)
    call(out)
    sync()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(out)
    for rep in range(4):
        fresh = torch.randint(0, 100, a.shape, dtype=torch.int8, device=dev).view(a.dtype)
        a.copy_(fresh)
        out_e = torch.zeros_like(out)
        call(out_e)
        sync()
        g.replay()
        sync()
        print(f"case: decode graph replay {kind} {rep}", flush=True)
        assert torch.equal(out.view(torch.uint8), out_e.view(torch.uint8))
        _ = (torch.randn(1024, device=dev) @ torch.randn(1024, device=dev))
