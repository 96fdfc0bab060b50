"""GPU parity of the FP8 delayed-scaling quantizer (the transformer-engine shim
ABI) against the CPU oracle.

Bars: the fp8 bits of the fused cast and the amax are bit-exact (f32 product
then the satfinite RNE encode; max is order-free); dequant is bit-exact after
the same RNE narrowing; the recipe follows the reference's published formula
exactly (scale = max_repr / max(history), one f32 division).  The recipe
cases restate crates/baracuda-transformer-engine/tests/recipe_*_smoke.rs.
"""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from oracle import oracle as O
from oracle.inputs import rng
from tests.gpu_util import sync

pytestmark = pytest.mark.gpu

FMTS = {"e4m3": P.Fp8Format.E4M3, "e5m2": P.Fp8Format.E5M2}
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _recipe(fmt, hist=4, scale=None):
    r = P.Fp8Recipe(FMTS[fmt], hist)
    if scale is not None:
        r.scale.fill_(scale)
    return r


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 7, 4099, 1 << 20])
def test_cast_amax_matches_oracle(gpu, fmt, dtype, n):
    print(f"case: te cast {fmt} {dtype} n={n}", flush=True)
    g = rng(n + 3)
    host = (g.standard_normal(n) * 20).astype(np.float32)
    if n >= 4099:   # out-of-range, inf and NaN inputs saturate / stay NaN, in both lanes of a pack
        host[:12] = [1e6, -1e6, np.inf, -np.inf, np.nan, -np.nan, 500.0, -70000.0, 138.0, 18000.0, 3e-9, -0.0]
    x = torch.from_numpy(host).to(dtype).to("cuda:0")
    r = _recipe(fmt, scale=3.25)
    out = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    P.Fp8CastPlan.select().run(x, out, r)
    sync()
    bits, amax = O.te_cast_amax(x.float().cpu().numpy(), 3.25, fmt)
    assert np.array_equal(out.cpu().numpy(), bits)
    hist = r.amax_history.cpu().numpy()
    assert hist[0] == amax and np.all(hist[1:] == 0)   # inf inputs make amax inf, as in the reference


def test_cast_unaligned_views_and_slot_accumulation(gpu):
    base = torch.randn(10001, device="cuda:0").to(torch.bfloat16)
    x = base[1:]                                  # 2-byte offset: element path
    obase = torch.zeros(10001, dtype=torch.uint8, device="cuda:0")
    out = obase[1:]
    r = _recipe("e4m3", hist=3)
    r.write_pos = 2
    P.Fp8CastPlan.select().run(x, out, r)
    x2 = torch.randn(64, device="cuda:0") * 100   # second cast into the same slot
    P.Fp8CastPlan.select().run(x2, torch.empty(64, dtype=torch.uint8, device="cuda:0"), r)
    sync()
    bits, a1 = O.te_cast_amax(x.float().cpu().numpy(), 1.0, "e4m3")
    assert np.array_equal(out.cpu().numpy(), bits) and obase[0].item() == 0
    a2 = float(x2.abs().max().item())
    assert r.amax_history.cpu().numpy().tolist() == [0.0, 0.0, max(a1, a2)]


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [256, 1003])
def test_dequant_matches_oracle(gpu, fmt, dtype, n):
    b = torch.from_numpy((np.arange(n) % 256).astype(np.uint8)).to("cuda:0")
    r = _recipe(fmt)
    r.scale_inv.fill_(0.3)
    y = torch.empty(n, dtype=dtype, device="cuda:0")
    P.Fp8DequantPlan.select().run(b, y, r)
    sync()
    want = torch.from_numpy(O.te_dequant_f32(b.cpu().numpy(), float(np.float32(0.3)), fmt)).to(dtype)
    got = y.cpu()
    both_nan = torch.isnan(got) & torch.isnan(want)
    iview = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(got[~both_nan].view(iview), want[~both_nan].view(iview))


def test_recipe_init_update_and_wrap(gpu):
    # recipe_amax_history_smoke.rs: history starts zero, write_pos wraps.
    r = _recipe("e4m3", hist=8)
    sync()
    assert r.amax_history.cpu().numpy().tolist() == [0.0] * 8
    assert r.scale_host() == 1.0 and r.scale_inv_host() == 1.0
    x = torch.randn(4096, device="cuda:0")
    out = torch.empty(4096, dtype=torch.uint8, device="cuda:0")
    for i in range(10):
        P.Fp8CastPlan.select().run(x * (i + 1), out, r)
        r.update_after_pass()
    assert r.write_pos == 10 % 8
    s, si = r.scale_host(), r.scale_inv_host()
    assert np.isfinite(s) and s > 0 and abs(s * si - 1) < 1e-5
    # The reference zeroes the consumed slot on every update.
    assert r.amax_history.cpu().numpy().tolist() == [0.0] * 8


@pytest.mark.parametrize("fmt,amax,expected", [("e4m3", 10.0, 44.8), ("e5m2", 100.0, 573.44)])
def test_recipe_scale_formula(gpu, fmt, amax, expected):
    # recipe_scale_compute_smoke.rs run_one: spike +amax at 512, -amax at 768.
    n = 1024
    host = np.sin(np.arange(n, dtype=np.float32) * np.float32(0.01)) * np.float32(amax * 0.1)
    host[512], host[768] = amax, -amax
    r = _recipe(fmt, hist=8)
    out = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    P.Fp8CastPlan.select().run(torch.from_numpy(host.astype(np.float32)).to("cuda:0"), out, r)
    r.update_after_pass()
    s, si = r.scale_host(), r.scale_inv_host()
    ws, wsi, _ = O.te_recipe_update([amax] + [0.0] * 7, fmt, 0)
    assert s == ws and si == wsi
    assert abs(s - expected) / expected < 1e-5 and abs(s * si - 1) < 1e-5
    # an empty history floors amax at 1: scale = max_repr
    r2 = _recipe(fmt, hist=8)
    r2.update_after_pass()
    assert r2.scale_host() == O.TE_MAX_REPR[fmt]


def test_quantizer_feeds_fp8_gemm(gpu):
    # Delayed scaling end to end: calibrate, cast A and B with the published
    # scales, run the FP8 GEMM with bf16 out and scale_inv_a * scale_inv_b;
    # the result tracks the bf16 product within e4m3 quantization error.
    m, n, k = 256, 512, 1024
    a = torch.randn(m, k, device="cuda:0").to(torch.bfloat16)
    b = torch.randn(n, k, device="cuda:0").to(torch.bfloat16)
    ra, rb = _recipe("e4m3", hist=1), _recipe("e4m3", hist=1)
    qa = torch.empty(m, k, dtype=torch.uint8, device="cuda:0")
    qb = torch.empty(n, k, dtype=torch.uint8, device="cuda:0")
    cast = P.Fp8CastPlan.select()
    for q, x, r in ((qa, a, ra), (qb, b, rb)):
        cast.run(x, q, r)
        r.update_after_pass()
        cast.run(x, q, r)
    d = torch.empty(m, n, dtype=torch.bfloat16, device="cuda:0")
    plan = P.Fp8GemmPlan.select(P.Fp8GemmDescriptor(m, n, k, output=P.ElementKind.Bf16))
    plan.run(qa, qb, d, scale_a=ra.scale_inv_host(), scale_b=rb.scale_inv_host())
    sync()
    ref = a.double() @ b.double().T
    rel = ((d.double() - ref).norm() / ref.norm()).item()
    assert rel < 0.05
    # and exactly what the oracle makes of the same fp8 bits
    exact = O.gemm_fp8_f64(qa.cpu().numpy(), qb.cpu().numpy(), "e4m3", rows=(0, 8)) * \
        (np.float32(ra.scale_inv_host()) * np.float32(rb.scale_inv_host()))
    got = d[:8].float().cpu().numpy()
    assert np.allclose(got, exact, rtol=2 ** -7, atol=1e-3 * np.abs(exact).max())


def test_cast_amax_keeps_larger_slot_value(gpu):
    # Workgroups whose max does not exceed the slot skip their atomic: a slot
    # already above every |x| keeps its value; one below it is raised to
    # exactly max|x|.
    x = torch.randn(1 << 22, device="cuda:0").to(torch.bfloat16)
    out = torch.empty(1 << 22, dtype=torch.uint8, device="cuda:0")
    want = float(x.float().abs().max().item())
    for start, expect in ((1000.0, 1000.0), (0.5, want), (want, want)):
        r = _recipe("e4m3", hist=2)
        r.amax_history.fill_(start)
        P.Fp8CastPlan.select().run(x, out, r)
        sync()
        assert r.amax_history.cpu().numpy().tolist() == [expect, start]


def test_cast_amax_beyond_2g_elements(gpu):
    # 2^31 + 29 bf16 elements (4 GiB in, 2 GiB out): 64-bit element indices
    # and, since n % 8 == 5, the scalar tail past element 2^31; sampled spans
    # (the last one ends at the final element) bit-exact, amax = max|x| exactly.
    n = (1 << 31) + 29
    assert n % 8 != 0
    print(f"case: te cast beyond 2^31 elements n={n}", flush=True)
    gen = torch.Generator(device="cuda:0").manual_seed(95)
    x = torch.empty(n, dtype=torch.bfloat16, device="cuda:0")
    x.normal_(generator=gen)
    out = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    r = _recipe("e4m3", hist=2, scale=2.5)
    P.Fp8CastPlan.select().run(x, out, r)
    sync()
    for s0 in (0, (1 << 30) + 8, (1 << 31) - 3, n - 4096, n - 13):
        e0 = min(s0 + 4096, n)
        bits, _ = O.te_cast_amax(x[s0:e0].float().cpu().numpy(), 2.5, "e4m3")
        assert np.array_equal(out[s0:e0].cpu().numpy(), bits), s0
    assert r.amax_history.cpu().numpy()[0] == float(x.abs().max().float().item())
    del x, out
