"""GPU parity of the int8 RCR last-rows path: when M % 256 is in [1, 128]
(N % 16 == 0, K % 128 == 0; above 64 rows only without the tail-split
workspace) and the last row of 256-row tiles would start another round of
tiles on the 256 CUs -- or M itself is at most 128 -- the whole tiles run
as usual and a streamed pass computes the last rows.  Every SKU family of
the RCR launch goes through it; outputs bit-exact against the oracle (int64
matmul for int32 out) on the rows around the boundary, the streamed rows
and sampled tile rows."""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from baracuda_amd.ffi import lib
from oracle import oracle as O
from oracle.inputs import int8_uniform, rng
from tests.gpu_util import dev, host_bits16, sync

pytestmark = pytest.mark.gpu

# (M, N, K).  M <= 128: the streamed pass alone, 1 / 16 / 33 / 64 / 100 /
# 128 rows (1, 2, 4 or 8 16-row fragments).  M > 256 at N = 16384 (64
# n-tiles): 4 tile rows fill one round exactly, so the fifth row of tiles
# would start a second round: 1 / 36 / 100 last rows.  K of 2 to 128 chunks
# of 64 bytes (each wave's batches, their remainder, or both).
SHAPES = [(1, 256, 384), (16, 4096, 4096), (33, 272, 640), (64, 1040, 1152), (100, 512, 4096),
          (128, 256, 8192), (1025, 16384, 128), (1060, 16384, 256), (1124, 16384, 128)]
# 2 to 16 last rows with K % 1024 == 0, K <= 8192: B streamed through LDS
# (gemm_s8_rcr_rows_dma_kernel; 1 to 8 chunks of 64 bytes per wave, 16 last
# rows under 4 tile rows); 17 to 32 rows (K % 512 == 0) take the staged
# kernel with two fragments.
DMA_SHAPES = [(1, 4096, 1024), (17, 512, 2048), (20, 1040, 3072), (32, 272, 8192), (1040, 16384, 1024),
              (2, 272, 1024), (9, 512, 2048), (1039, 16384, 3072)]
SHAPES += DMA_SHAPES
# One last row with K % 1024 == 0: the dot4 row kernel (gemm_s8_rcr_row1_kernel;
# 1 or 2 kilobytes per batch, the row under 4 tile rows).
ROW1_SHAPES = [(1, 512, 2048), (1, 1040, 3072), (1, 4096, 4096), (1025, 16384, 2048)]
SHAPES += ROW1_SHAPES
# 17 (9 for N >= 6144) to 128 last rows with K % 512 == 0: A and B streamed through LDS in K
# stages (gemm_s8_rcr_rows_staged_kernel; 2, 4 or 8 fragments, 1 to 16
# stages, the last-rows pass under 4 tile rows), 16 columns per workgroup
# below N = 6144, 32 from 6144 (16 / 20 / 64 / 128 rows), 64 from 12288 (9 / 17 rows;
# 36 and 100 under the tile rows at N = 16384).
STAGED_SHAPES = [(17, 256, 512), (31, 1040, 1536), (33, 512, 512), (65, 272, 1024), (97, 1040, 2560), (1060, 16384, 1536), (1124, 16384, 512),
                 (20, 6144, 1024), (64, 8192, 512), (128, 6144, 1024), (17, 12288, 512),
                 (9, 14336, 1024), (16, 6144, 512),
                 # 33-128 rows below N = 6144 in row blocks (mfma2::last_rows_blocks):
                 # 64-row blocks of 32 columns, 32-row blocks of 32 columns, 3 blocks
                 (100, 4096, 1024), (128, 2048, 512), (48, 4096, 512), (90, 3072, 512),
                 # 11-16 rows below N = 6144: one fragment, 8 of 16 waves multiplying
                 (11, 1040, 1024), (16, 4096, 2048),
                 # 6-8 rows at 64 columns (N >= 12288): one fragment
                 (6, 12288, 1024), (8, 14336, 512)]
SHAPES += STAGED_SHAPES


def _rows(m):
    # rows checked: around the tile / streamed boundary, the streamed rows,
    # and a few tile rows
    m0 = m - m % 256 if m > 256 else 0
    rows = set(range(max(0, m0 - 2), m)) | set(int(r) for r in rng(m).integers(0, m, 6))
    return sorted(rows)


@pytest.mark.parametrize("shape", SHAPES)
def test_rows_path_i32_s8_w8a8(gpu, shape):
    m, n, k = shape
    print(f"case: rows path {shape}", flush=True)
    g = rng(m * 7 + n + k)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    rows = _rows(m)
    assert P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16)).workspace_size() == 0 \
        or m % 256 > 64
    d = torch.full((m, n), -7, dtype=torch.int32, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.I32)).run(dev(a), dev(b), d)
    sync()
    got = d.cpu().numpy()
    assert np.array_equal(got[rows], a[rows].astype(np.int64) @ b.astype(np.int64).T)

    c = int8_uniform(g, (m, n))
    d8 = torch.full((m, n), 99, dtype=torch.int8, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k)).run(dev(a), dev(b), d8, c=dev(c), alpha=0.003, beta=0.5)
    sync()
    assert np.array_equal(d8.cpu().numpy()[rows], O.gemm_s8_rcr_s8(a[rows], b, 0.003, 0.5, c[rows]))

    sa = g.uniform(0.005, 0.02, m).astype(np.float32)
    sw = g.uniform(0.001, 0.01, n).astype(np.float32)
    dw = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16)).run(
        dev(a), dev(b), dw, scale_a=dev(sa), scale_b=dev(sw))
    sync()
    gw = host_bits16(dw)
    for r in rows:
        assert np.array_equal(gw[r], O.gemm_w8a8_bf16(a, b, sa, sw, rows=(r, r + 1), nthreads=8)[0]), r


@pytest.mark.parametrize("shape", [SHAPES[1], SHAPES[4], SHAPES[7], DMA_SHAPES[1], DMA_SHAPES[4], STAGED_SHAPES[0], STAGED_SHAPES[4], STAGED_SHAPES[6], STAGED_SHAPES[8], STAGED_SHAPES[10], ROW1_SHAPES[0], ROW1_SHAPES[3], DMA_SHAPES[6]])
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
    rows = _rows(m)
    assert np.array_equal(d.cpu().numpy()[rows], O.gemm_s8_epi(a[rows], b, "rcr", 0.004, 0.25, c[rows], bias, "gelu"))


@pytest.mark.parametrize("shape", [SHAPES[2], SHAPES[3], SHAPES[5], SHAPES[6], DMA_SHAPES[2], DMA_SHAPES[3], STAGED_SHAPES[1], STAGED_SHAPES[3], STAGED_SHAPES[5], ROW1_SHAPES[1]])
def test_rows_path_quantized_linear_f32_f64(gpu, shape):
    # f32: y = (sa*sw)*acc in f32; f64: f64 scales narrowed to f32, the same
    # product, widened (compose.cu:27-28).
    m, n, k = shape
    print(f"case: rows path quantized_linear {shape}", flush=True)
    g = rng(m + n + 5 * k)
    a, w = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    rows = _rows(m)
    acc = (a[rows].astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
    stream = torch.cuda.current_stream().cuda_stream
    sa = g.uniform(0.005, 0.02, m).astype(np.float32)
    sw = g.uniform(0.001, 0.01, n).astype(np.float32)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    tw, ta, tsa, tsw = dev(w), dev(a), dev(sa), dev(sw)
    assert lib().quantized_linear_w8a8_f32_gfx950_run(m, n, k, tw.data_ptr(), ta.data_ptr(), tsa.data_ptr(),
                                                      tsw.data_ptr(), out.data_ptr(), None, 0, stream) == 0
    sync()
    assert np.array_equal(out.cpu().numpy()[rows], (sa[rows][:, None] * sw[None, :]).astype(np.float32) * acc)
    sa64, sw64 = g.uniform(0.005, 0.02, m), g.uniform(0.001, 0.01, n)
    out64 = torch.empty((m, n), dtype=torch.float64, device="cuda:0")
    tsa64, tsw64 = dev(sa64), dev(sw64)
    assert lib().quantized_linear_w8a8_f64_gfx950_run(m, n, k, tw.data_ptr(), ta.data_ptr(), tsa64.data_ptr(),
                                                      tsw64.data_ptr(), out64.data_ptr(), None, 0, stream) == 0
    sync()
    want64 = ((sa64[rows].astype(np.float32)[:, None] * sw64.astype(np.float32)[None, :]).astype(np.float32)
              * acc).astype(np.float64)
    assert np.array_equal(out64.cpu().numpy()[rows], want64)


def test_rows_path_with_and_without_split_workspace(gpu):
    # 100 last rows at M = 1124, N = 16384, K = 1152 (not a multiple of the
    # staged kernel's 512-byte stages): with the tail-split workspace the
    # split runs, without it the last-rows pass; both equal the oracle rows.
    m, n, k = 1124, 16384, 1152
    print("case: rows path vs tail split", flush=True)
    g = rng(77)
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.I32))
    assert plan.workspace_size() > 0
    outs = []
    for ws in (None, torch.empty(plan.workspace_size(), dtype=torch.uint8, device="cuda:0")):
        d = torch.full((m, n), -7, dtype=torch.int32, device="cuda:0")
        plan.run(dev(a), dev(b), d, workspace=ws)
        sync()
        outs.append(d.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    rows = _rows(m)
    assert np.array_equal(outs[0][rows], a[rows].astype(np.int64) @ b.astype(np.int64).T)


@pytest.mark.parametrize("shape", [(7, 512, 2048), (30, 4096, 1024), (100, 1024, 2048), (60, 512, 1536), (1, 1024, 2048),
                                   (12, 4096, 1024), (8, 12288, 1024), (200, 2048, 1024)])
def test_rows_dma_padded_leading_dimensions(gpu, shape):
    # A, B and D views with row pitches past K / N (16-byte multiples): the
    # LDS-streamed kernels address rows by ldb and A rows by lda, the
    # epilogue D rows by ldd (one-fragment blocks at 12 x 4096 and 8 x 12288,
    # 64-row blocks of a small grid at 200 x 2048); columns past N untouched.
    m, n, k = shape
    print(f"case: rows dma padded ld {shape}", flush=True)
    g = rng(m + n + k + 3)
    a_full, b_full = int8_uniform(g, (m, k + 64)), int8_uniform(g, (n, k + 128))
    ta, tb = dev(a_full)[:, :k], dev(b_full)[:, :k]
    d_full = torch.full((m, n + 32), -7, dtype=torch.int32, device="cuda:0")
    P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.I32)).run(ta, tb, d_full[:, :n])
    sync()
    want = a_full[:, :k].astype(np.int64) @ b_full[:, :k].astype(np.int64).T
    got = d_full.cpu().numpy()
    assert np.array_equal(got[:, :n], want)
    assert np.all(got[:, n:] == -7)
