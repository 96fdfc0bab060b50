"""GPU parity of the float MoE grouped GEMM (the reference's moe_wmma ABI,
bf16 / f16) against the CPU oracle.

Bar: with f32 accumulation of exact 16-bit products, each output is within
one ulp of its type (bf16 / f16) of the exact value plus the MFMA's f32
summation error, 2^-20 * sum_k |x*w| (* |topk weight|).  The reference's own
smoke test (moe_wmma_smoke.rs) allows 3% per cell on its fixture; here its
fixture is held to the tighter bar.
"""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from oracle import oracle as O
from oracle.inputs import moe_routing, rng
from tests.gpu_util import dev, sync

pytestmark = pytest.mark.gpu

TDT = {"bf16": torch.bfloat16, "f16": torch.float16}
KIND = {"bf16": P.ElementKind.Bf16, "f16": P.ElementKind.F16}


def _ulp(v, t):
    a = np.abs(v).astype(np.float64)
    if t == "bf16":
        e = np.floor(np.log2(np.where(a > 0, a, 2.0 ** -126)))
        return np.exp2(np.maximum(e, -126) - 7)
    e = np.floor(np.log2(np.where(a > 0, a, 2.0 ** -14)))
    return np.exp2(np.maximum(e, -14) - 10)


def _run(t, x, w, sid, eid, topk, tw, size_rows, is_prefill=True):
    E, n, k = w.shape
    tokens = x.shape[0] if tw is None else x.shape[0] // topk
    plan = P.MoePlan.select(P.MoeDescriptor(tokens, E, topk, k, n, element=KIND[t], is_prefill=is_prefill))
    dx = torch.from_numpy(x).to(TDT[t]).to("cuda:0")
    dw = torch.from_numpy(w).to(TDT[t]).to("cuda:0")
    out = torch.zeros((size_rows, n), dtype=TDT[t], device="cuda:0")
    counts = torch.zeros(E, dtype=torch.int32, device="cuda:0")
    offs = torch.zeros(E + 1, dtype=torch.int32, device="cuda:0")
    plan.run(dx, dw, dev(sid), dev(eid), out, counts, offs, topk_weights=None if tw is None else dev(tw))
    sync()
    c_ref, o_ref = O.moe_expert_offsets(eid, E)
    assert np.array_equal(counts.cpu().numpy(), c_ref) and np.array_equal(offs.cpu().numpy(), o_ref)
    xf = dx.float().cpu().numpy()
    wf = dw.float().cpu().numpy()
    exact = O.moe_grouped_f64(xf, wf, sid, o_ref, topk, tw, out_rows=size_rows)
    absx = O.moe_grouped_f64(np.abs(xf), np.abs(wf), sid, o_ref, topk,
                             None if tw is None else np.abs(tw), out_rows=size_rows)
    return out.float().cpu().numpy(), exact, absx


def _check(got, exact, absx, t):
    rows = ~np.isnan(exact[:, 0])
    g, e, a = got[rows], exact[rows], absx[rows]
    tol = _ulp(e, t) + 2.0 ** -20 * a
    bad = np.abs(g - e) > tol
    assert not bad.any(), f"{bad.sum()} cells off; worst {np.abs(g - e)[bad].max()}"


@pytest.mark.parametrize("t", ["f16", "bf16"])
def test_reference_smoke_fixture(gpu, t):
    # moe_wmma_smoke.rs:36-135: T=4 tokens, 2 experts, top_k=1, DM=16, DE=32,
    # acts (i*0.1 + j*0.01), w[e,n,k] = (e+1)*0.001*(n-k), token t -> expert t%2,
    # topk weight 0.6.
    T, NE, DM, DE = 4, 2, 16, 32
    x = (0.1 * np.arange(T)[:, None] + 0.01 * np.arange(DM)[None, :]).astype(np.float32)
    w = ((np.arange(NE)[:, None, None] + 1) * 0.001 *
         (np.arange(DE)[None, :, None] - np.arange(DM)[None, None, :])).astype(np.float32)
    order = sorted(range(T), key=lambda tt: tt % NE)
    sid = np.array(order, np.int32)
    eid = np.array([tt % NE for tt in order], np.int32)
    tw = np.full(T, 0.6, np.float32)
    got, exact, absx = _run(t, x, w, sid, eid, 1, tw, T)
    _check(got, exact, absx, t)
    # the reference test's own 3% bar, on the reference's own f32 CPU sum
    assert np.all(np.abs(got - exact) <= 0.03 * np.maximum(np.abs(exact), 1e-3))


@pytest.mark.parametrize("topk_w", [False, True])
@pytest.mark.parametrize("t", ["bf16", "f16"])
@pytest.mark.parametrize("shape", [(64, 4, 2, 96, 100), (512, 8, 2, 512, 512), (300, 8, 2, 256, 1024),
                                   (1024, 16, 4, 256, 256), (1, 8, 2, 512, 512), (16, 8, 2, 6144, 256),
                                   (32, 16, 2, 512, 1024)])
def test_random_routing(gpu, shape, t, topk_w):
    # Zipf routing; (512, ..., 512, 512) and (1024, ..., 256, 256) take the
    # LDS-DMA path (K a multiple of 64 elements, N of 256), the others the
    # general path (K tail, N tail); size_m = 2 / 32 / 64 with K a multiple
    # of 256 elements the decode-sized pass (moe_rows_staged_kernel).
    tokens, E, topk, n, k = shape
    print(f"case: moe_wmma {t} topk_w={topk_w} {shape}", flush=True)
    sid, eid = moe_routing(tokens, E, topk, seed=tokens + n)
    g = rng(tokens + k)
    size_m = tokens * topk
    x = g.standard_normal((size_m if topk_w else tokens, k)).astype(np.float32)
    w = (g.standard_normal((E, n, k)) * 0.1).astype(np.float32)
    tw = g.uniform(0.1, 1.0, size_m).astype(np.float32) if topk_w else None
    got, exact, absx = _run(t, x, w, sid, eid, topk, tw, size_m, is_prefill=tokens > 256)
    _check(got, exact, absx, t)


@pytest.mark.parametrize("t", ["bf16", "f16"])
def test_partial_tile_boundaries(gpu, t):
    # LDS-DMA path with last tiles of 1, 128 and 129 rows and an empty expert.
    counts = [257, 128, 0, 129]
    tokens = sum(counts)
    pair_expert = np.repeat(np.arange(len(counts), dtype=np.int32), counts)
    rng(13).shuffle(pair_expert)
    sid = np.argsort(pair_expert, kind="stable").astype(np.int32)
    eid = pair_expert[sid].astype(np.int32)
    g = rng(14)
    x = g.standard_normal((tokens, 256)).astype(np.float32)
    w = (g.standard_normal((len(counts), 256, 256)) * 0.1).astype(np.float32)
    got, exact, absx = _run(t, x, w, sid, eid, 1, None, tokens, is_prefill=True)
    _check(got, exact, absx, t)
