"""GPU parity of the decode kernels: gemv_s8w_m1, gemv_dense_m1 and gather_rows,
including hipGraph capture + replay (capture_replay_gather_gemv.rs)."""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from baracuda_amd.ffi import lib
from oracle import oracle as O
from oracle.inputs import int8_uniform, rng
from tests.gpu_util import bf16_ulp, dev, host_bits16, sync

pytestmark = pytest.mark.gpu
GOLD = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def _gemv_inputs(n, k, seed=4):
    g = rng(seed)
    w = int8_uniform(g, (n, k))
    scale = g.uniform(0.001, 0.01, n).astype(np.float32)
    xb = O.f32_to_bf16_bits_fast(g.standard_normal(k).astype(np.float32))
    return w, scale, xb


def _gemv_check(got_bits, w, scale, xb):
    # <= 1 bf16 ulp of the exact value; absolute floor 1e-6 * scale * sum|x*w|
    # for outputs whose sum cancels.
    acc = O.gemv_s8w_m1_f64(xb, w, nthreads=8)
    exact = acc * scale.astype(np.float64)
    got = O.bf16_bits_to_f32(got_bits).astype(np.float64)
    absum = np.abs(w.astype(np.float64)) @ np.abs(O.bf16_bits_to_f32(xb).astype(np.float64)) * scale
    err = np.abs(got - exact)
    assert np.all(err <= bf16_ulp(exact) + 1e-6 * absum), err.max()


def _gemv_run(w, scale, xb):
    n, k = w.shape
    d = torch.empty(n, dtype=torch.bfloat16, device="cuda:0")
    x = dev(xb).view(torch.bfloat16)
    P.GemvS8wPlan.select(n, k).run(x, dev(w), dev(scale), d)
    sync()
    return host_bits16(d)


@pytest.mark.parametrize("shape", [(14336, 4096), (4096, 14336), (1, 1024), (77, 3000), (1000, 17), (5, 5120),
                                   (3, 12288)])
def test_gemv_s8w(gpu, shape):
    print(f"case: gemv_s8w {shape}", flush=True)
    w, scale, xb = _gemv_inputs(*shape)
    _gemv_check(_gemv_run(w, scale, xb), w, scale, xb)


def test_gemv_s8w_empty_reduction(gpu):
    # K == 0 with valid (non-null) buffers: every output is bf16(0 * scale) = 0.
    n = 33
    w = torch.zeros((n, 1), dtype=torch.int8, device="cuda:0")    # non-null buffers, K = 0
    x = torch.zeros(1, dtype=torch.bfloat16, device="cuda:0")
    d = torch.full((n,), 5.0, dtype=torch.bfloat16, device="cuda:0")
    scale = torch.ones(n, device="cuda:0")
    st = lib().gemv_s8w_m1_bf16_gfx950_run(n, 0, x.data_ptr(), w.data_ptr(), 1,
                                           scale.data_ptr(), d.data_ptr(),
                                           None, 0, torch.cuda.current_stream().cuda_stream)
    sync()
    assert st == 0 and torch.all(d == 0)


def test_gemv_s8w_graph_replay_bit_identical(gpu):
    n, k = 14336, 4096
    w, scale, xb = _gemv_inputs(n, k)
    wd, sd, x = dev(w), dev(scale), dev(xb).view(torch.bfloat16)
    d = torch.zeros(n, dtype=torch.bfloat16, device="cuda:0")
    plan = P.GemvS8wPlan.select(n, k)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        plan.run(x, wd, sd, d)
    torch.cuda.synchronize()
    warm = host_bits16(d).copy()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run(x, wd, sd, d)
    for rep in range(4):
        d.fill_(0)
        graph.replay()
        sync()
        assert np.array_equal(host_bits16(d), warm), rep
    _gemv_check(warm, w, scale, xb)


_TORCH = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


@pytest.mark.parametrize("tag", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", [(4096, 4096, 1, False, 0.0), (37, 19, 3, True, 0.25), (300, 1000, 4, False, 0.5),
                                  (512, 1000, 3, True, 0.25), (256, 64, 2, False, 0.5), (96, 7, 1, False, 0.0)])
def test_gemv_dense_m1(gpu, tag, case):
    # gemv_dense_smoke.rs: f32 rel 1e-4, bf16 rel 1.6e-2 (f16 taken as 2e-3),
    # GQA broadcast (stride_b = 0), strided batch, beta, inter-slot gaps untouched.
    n, k, batch, bcast, beta = case
    print(f"case: gemv_dense {tag} {case}", flush=True)
    g = rng(n + k + batch)
    dt = _TORCH[tag]
    stride_a, stride_d, ldb = k + 3, n + 5, n
    stride_b = 0 if bcast else k * ldb
    a = torch.from_numpy(g.standard_normal(batch * stride_a).astype(np.float32)).to(dt)
    b = torch.from_numpy(g.standard_normal(max(1, (1 if bcast else batch)) * k * ldb).astype(np.float32) / 8).to(dt)
    d0 = torch.from_numpy(g.standard_normal(batch * stride_d).astype(np.float32)).to(dt)
    d = d0.clone().cuda()
    plan = P.GemvDensePlan.select(P.GemvDenseDescriptor(n=n, k=k, batch=batch), dt)
    plan.can_implement(k, ldb, n, stride_a, stride_b, stride_d)
    plan.run(a.cuda(), b.cuda(), d, lda=k, stride_a=stride_a, ldb=ldb, stride_b=stride_b, ldd=n,
             stride_d=stride_d, alpha=0.75, beta=beta)
    sync()
    want = O.gemv_dense_m1_f64(a.double().numpy(), b.double().numpy(), d0.double().numpy(), n, k, batch,
                               stride_a, ldb, stride_b, stride_d, 0.75, beta)
    got = d.cpu().double().numpy()
    rel = {"f32": 1e-4, "f16": 2e-3, "bf16": 1.6e-2}[tag]
    for gi in range(batch):
        sl = slice(gi * stride_d, gi * stride_d + n)
        scale = np.abs(want[sl]).max()
        assert np.allclose(got[sl], want[sl], rtol=rel, atol=rel * scale), gi
        gap = slice(gi * stride_d + n, (gi + 1) * stride_d)
        assert np.array_equal(got[gap], d0.double().numpy()[gap])


@pytest.mark.parametrize("tag", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", [(4096, 4096, 1, False, 0.0), (512, 4096, 3, True, 0.25), (2048, 1000, 2, False, 0.5),
                                  (8192, 257, 1, False, 0.0)])
def test_gemv_dense_m1_split_workspace(gpu, tag, case):
    # The optional-workspace split-K path (contiguous B row spans, fixed-order
    # partial sums): same tolerances against the f64 reference, strided batch,
    # broadcast B, beta, gaps between batch slots untouched.
    n, k, batch, bcast, beta = case
    print(f"case: gemv_dense split {tag} {case}", flush=True)
    g = rng(7 * n + k + batch)
    dt = _TORCH[tag]
    stride_a, stride_d, ldb = k + 3, n + 5, n
    stride_b = 0 if bcast else k * ldb
    a = torch.from_numpy(g.standard_normal(batch * stride_a).astype(np.float32)).to(dt)
    b = torch.from_numpy(g.standard_normal(max(1, (1 if bcast else batch)) * k * ldb).astype(np.float32) / 8).to(dt)
    d0 = torch.from_numpy(g.standard_normal(batch * stride_d).astype(np.float32)).to(dt)
    d = d0.clone().cuda()
    plan = P.GemvDensePlan.select(P.GemvDenseDescriptor(n=n, k=k, batch=batch), dt)
    wsb = plan.workspace_size()
    rows = 8 if tag == "f32" else 16   # rows per slice
    assert wsb == batch * ((k + rows - 1) // rows) * n * 4
    ws = torch.full((wsb // 4,), float("nan"), dtype=torch.float32, device="cuda:0")
    plan.run(a.cuda(), b.cuda(), d, lda=k, stride_a=stride_a, ldb=ldb, stride_b=stride_b, ldd=n,
             stride_d=stride_d, alpha=0.75, beta=beta, workspace=ws)
    sync()
    want = O.gemv_dense_m1_f64(a.double().numpy(), b.double().numpy(), d0.double().numpy(), n, k, batch,
                               stride_a, ldb, stride_b, stride_d, 0.75, beta)
    got = d.cpu().double().numpy()
    rel = {"f32": 1e-4, "f16": 2e-3, "bf16": 1.6e-2}[tag]
    for gi in range(batch):
        sl = slice(gi * stride_d, gi * stride_d + n)
        scale = np.abs(want[sl]).max()
        assert np.allclose(got[sl], want[sl], rtol=rel, atol=rel * scale), gi
        gap = slice(gi * stride_d + n, (gi + 1) * stride_d)
        assert np.array_equal(got[gap], d0.double().numpy()[gap])


@pytest.mark.parametrize("tag", ["f32", "bf16"])
def test_gemv_dense_split_bit_stable_and_capturable(gpu, tag):
    # Fixed partial and reduction orders: launches and graph replays agree bit for bit.
    n, k = 4096, 4096
    dt = _TORCH[tag]
    a = torch.randn(k, device="cuda:0").to(dt)
    b = torch.randn(k * n, device="cuda:0").to(dt)
    plan = P.GemvDensePlan.select(P.GemvDenseDescriptor(n=n, k=k), dt)
    ws = torch.empty(plan.workspace_size(), dtype=torch.uint8, device="cuda:0")
    run = lambda d: plan.run(a, b, d, lda=k, stride_a=0, ldb=n, stride_b=0, ldd=n, stride_d=0, workspace=ws)  # noqa: E731
    outs = []
    for _ in range(2):
        d = torch.empty(n, dtype=dt, device="cuda:0")
        run(d)
        outs.append(d)
    dg = torch.empty(n, dtype=dt, device="cuda:0")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(dg)
    iv = torch.int32 if tag == "f32" else torch.int16
    for _ in range(3):
        dg.fill_(0)
        g.replay()
        sync()
        assert torch.equal(outs[0].view(iv), outs[1].view(iv)) and torch.equal(outs[0].view(iv), dg.view(iv))


@pytest.mark.parametrize("tag", ["f32", "bf16"])
def test_gemv_dense_bit_stable_across_launches(gpu, tag):
    # The reduction order is fixed: two launches (and a graph replay) agree bit for bit.
    n, k = 4096, 4096
    dt = _TORCH[tag]
    a = torch.randn(k, device="cuda:0").to(dt)
    b = torch.randn(k * n, device="cuda:0").to(dt)
    plan = P.GemvDensePlan.select(P.GemvDenseDescriptor(n=n, k=k), dt)
    outs = []
    for _ in range(2):
        d = torch.empty(n, dtype=dt, device="cuda:0")
        plan.run(a, b, d, lda=k, stride_a=0, ldb=n, stride_b=0, ldd=n, stride_d=0)
        outs.append(d)
    dg = torch.empty(n, dtype=dt, device="cuda:0")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        plan.run(a, b, dg, lda=k, stride_a=0, ldb=n, stride_b=0, ldd=n, stride_d=0)
    g.replay()
    sync()
    iv = torch.int32 if tag == "f32" else torch.int16
    assert torch.equal(outs[0].view(iv), outs[1].view(iv)) and torch.equal(outs[0].view(iv), dg.view(iv))


def test_gemv_dense_beta0_never_reads_d(gpu):
    n, k = 256, 64
    a = torch.ones(k, device="cuda:0")
    b = torch.ones(k * n, device="cuda:0")
    d = torch.full((n,), float("nan"), device="cuda:0")
    P.GemvDensePlan.select(P.GemvDenseDescriptor(n=n, k=k), torch.float32).run(
        a, b, d, lda=k, stride_a=0, ldb=n, stride_b=0, ldd=n, stride_d=0, alpha=1.0, beta=0.0)
    sync()
    assert torch.all(d == k)


# ---- gather_rows ---------------------------------------------------------------
def test_gather_rows_capture_replay_golden(gpu):
    # capture_replay_gather_gemv.rs:54-117: warm launch + 4 graph replays == [1,2,3,4].
    z = np.load(GOLD / "wte_gather.npz")
    table = dev(z["table"])
    idx = dev(z["idx"].view(np.int32)).view(torch.uint32)
    dest = torch.zeros((1, 4), dtype=torch.float32, device="cuda:0")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        P.gather_rows(dest, table, idx)
    torch.cuda.synchronize()
    assert np.array_equal(dest.cpu().numpy(), z["expected"])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        P.gather_rows(dest, table, idx)
    for rep in range(4):
        graph.replay()
        sync()
        assert np.array_equal(dest.cpu().numpy(), z["expected"]), rep


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_gather_rows_oob_and_ragged(gpu, dt):
    g = rng(31)
    V, H = 50, 36 if dt != torch.float32 else 37     # 72-byte / 148-byte rows: element path
    table = torch.from_numpy(g.standard_normal((V, H)).astype(np.float32)).to(dt)
    idx = np.array([3, 49, 50, 2 ** 32 - 1, 0, 3], np.uint32)
    dest = torch.full((idx.size, H), 7, dtype=dt, device="cuda:0")
    P.gather_rows(dest, table.cuda(), dev(idx.view(np.int32)).view(torch.uint32))
    sync()
    tb = table.view(torch.int16 if dt != torch.float32 else torch.int32).numpy()
    want = O.gather_rows(tb, idx)
    got = dest.cpu().view(torch.int16 if dt != torch.float32 else torch.int32).numpy()
    assert np.array_equal(got, want)


def test_gather_rows_config4_bf16_table(gpu):
    # BASELINE.json config 4b: bf16 [128256, 4096] ~ N(0, 0.02), n in {1, 8, 64}.
    V, H = 128256, 4096
    gen = torch.Generator(device="cuda:0").manual_seed(4)
    table = (torch.randn((V, H), generator=gen, device="cuda:0") * 0.02).to(torch.bfloat16)
    g = rng(41)
    for n in (1, 8, 64):
        print(f"case: gather bf16 n={n}", flush=True)
        idx = g.integers(0, V, n).astype(np.uint32)
        idx[0] = V - 1
        dest = torch.empty((n, H), dtype=torch.bfloat16, device="cuda:0")
        P.gather_rows(dest, table, dev(idx.view(np.int32)).view(torch.uint32))
        sync()
        rows = table[torch.from_numpy(idx.astype(np.int64)).cuda()].cpu().view(torch.int16).numpy()
        # oracle on the gathered rows only (remapped indices 0..n-1), bit-exact
        want = O.gather_rows(rows, np.arange(n, dtype=np.uint32))
        assert np.array_equal(dest.cpu().view(torch.int16).numpy(), want)


def test_gemv_s8w_weights_beyond_2gib(gpu):
    # W is 262152 x 8192 int8 (2 GiB + 64 KiB): byte offsets past 2^31 need
    # 64-bit row addressing; sampled rows (the last 8 lie wholly past 2^31)
    # within 1 bf16 ulp of the exact f64 value.
    n, k = 262152, 8192
    assert (n - 1) * k > 2 ** 31
    print(f"case: gemv_s8w beyond 2 GiB {n}x{k}", flush=True)
    gen = torch.Generator(device="cuda:0").manual_seed(91)
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda:0", generator=gen)
    scale = (torch.rand(n, device="cuda:0", generator=gen) * 0.009 + 0.001)
    x = torch.randn(k, device="cuda:0", generator=gen).to(torch.bfloat16)
    d = torch.empty(n, dtype=torch.bfloat16, device="cuda:0")
    P.GemvS8wPlan.select(n, k).run(x, w, scale, d)
    sync()
    rows = [0, 1, 131071, 262143, 262144, 262148, n - 1] + list(rng(92).integers(0, n, 4))
    xb = x.cpu().view(torch.int16).numpy().view(np.uint16)
    got = host_bits16(d)[rows]
    wr = w[rows].cpu().numpy()
    _gemv_check(got, wr, scale[rows].cpu().numpy(), xb)
    del w
