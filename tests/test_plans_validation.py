"""Host-side operand validation of the Plan mirror (no GPU): every 1-D operand
the kernels index as dense memory must be a contiguous 1-D vector of the
stated length, so a strided view raises InvalidProblem before any launch
instead of being read or written as if it were dense."""
import pytest
import torch

from baracuda_amd import plans as P


def _strided(n, dtype):
    """A length-n view with stride 2 (column 0 of an [n, 2] tensor)."""
    return torch.zeros((n, 2), dtype=dtype)[:, 0]


def test_w8a8_strided_scales_rejected():
    m = n = k = 256
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16))
    a = torch.zeros((m, k), dtype=torch.int8)
    w = torch.zeros((n, k), dtype=torch.int8)
    d = torch.empty((m, n), dtype=torch.bfloat16)
    good_a, good_b = torch.ones(m), torch.ones(n)
    with pytest.raises(P.InvalidProblem):
        plan.run(a, w, d, scale_a=_strided(m, torch.float32), scale_b=good_b, stream=0)
    with pytest.raises(P.InvalidProblem):
        plan.run(a, w, d, scale_a=good_a, scale_b=_strided(n, torch.float32), stream=0)
    with pytest.raises(P.InvalidProblem):    # [M, 1] is not a 1-D vector
        plan.run(a, w, d, scale_a=good_a.view(m, 1), scale_b=good_b, stream=0)
    with pytest.raises(P.InvalidProblem):    # missing scale
        plan.run(a, w, d, scale_a=None, scale_b=good_b, stream=0)


def test_gemv_s8w_strided_vectors_rejected():
    n, k = 64, 128
    plan = P.GemvS8wPlan.select(n, k)
    w = torch.zeros((n, k), dtype=torch.int8)
    x = torch.zeros(k, dtype=torch.bfloat16)
    sc = torch.ones(n)
    d = torch.empty(n, dtype=torch.bfloat16)
    for args in ((_strided(k, torch.bfloat16), w, sc, d), (x, w, _strided(n, torch.float32), d),
                 (x, w, sc, _strided(n, torch.bfloat16))):
        with pytest.raises(P.InvalidProblem):
            plan.run(*args, stream=0)


def test_quantizer_strided_scale_rejected():
    x = torch.zeros((8, 64), dtype=torch.float32)
    q = torch.empty((8, 64), dtype=torch.int8)
    with pytest.raises(P.InvalidProblem):
        P.dynamic_range_quantize_per_token_sym(x, _strided(8, torch.float32), q, stream=0)


def test_bias_must_be_1d_contiguous():
    m = n = k = 128
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, epilogue=P.EpilogueKind.Bias))
    a = torch.zeros((m, k), dtype=torch.int8)
    b = torch.zeros((n, k), dtype=torch.int8)
    d = torch.empty((m, n), dtype=torch.int8)
    with pytest.raises(P.InvalidProblem):
        plan.run(a, b, d, bias=_strided(n, torch.float32), stream=0)


def test_moe_strided_routing_rejected():
    E, topk, tokens, n, k = 4, 2, 16, 256, 128
    plan = P.MoeS8GroupedPlan(E, topk, tokens * topk, n, k)   # select() needs no GPU either, but
    x = torch.zeros((tokens, k), dtype=torch.int8)            # the validation under test is run()'s
    w = torch.zeros((E, n, k), dtype=torch.int8)
    out = torch.empty((tokens * topk, n), dtype=torch.bfloat16)
    sid = torch.zeros(tokens * topk, dtype=torch.int32)
    eid = torch.zeros(tokens * topk, dtype=torch.int32)
    cnt = torch.empty(E, dtype=torch.int32)
    off = torch.empty(E + 1, dtype=torch.int32)
    sa, sw = torch.ones(tokens), torch.ones(E * n)
    good = dict(sorted_token_ids=sid, expert_ids=eid, expert_counts=cnt, expert_offsets=off,
                scale_a=sa, scale_w=sw)
    bad = {"sorted_token_ids": _strided(tokens * topk, torch.int32),
           "expert_ids": _strided(tokens * topk, torch.int32),
           "expert_counts": _strided(E, torch.int32), "expert_offsets": _strided(E + 1, torch.int32),
           "scale_a": _strided(tokens, torch.float32), "scale_w": _strided(E * n, torch.float32)}
    for key, val in bad.items():
        kw = dict(good)
        kw[key] = val
        with pytest.raises(P.InvalidProblem):
            plan.run(x, w, out=out, stream=0, **kw)
    with pytest.raises(P.InvalidProblem):
        plan.run(x, w, out=out, topk_weights=_strided(tokens * topk, torch.float32), stream=0, **good)


def test_host_tensors_rejected_before_launch():
    # Valid shapes and dtypes, but host memory: rejected before any kernel
    # would dereference a host address.
    m = n = k = 256
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.I32))
    a = torch.zeros((m, k), dtype=torch.int8)
    b = torch.zeros((n, k), dtype=torch.int8)
    d = torch.empty((m, n), dtype=torch.int32)
    with pytest.raises(P.InvalidProblem, match="GPU"):
        plan.run(a, b, d, stream=0)
    gp = P.GemvDensePlan.select(P.GemvDenseDescriptor(n=64, k=64), torch.float32)
    with pytest.raises(P.InvalidProblem, match="GPU"):
        gp.run(torch.ones(64), torch.ones(64 * 64), torch.empty(64), lda=64, stride_a=0, ldb=64, stride_b=0,
               ldd=64, stride_d=0, stream=0)
