"""Seeded random-shape sweep on the grid of the last-rows kernels (GPU parity).

The shapes of test_gpu_sweep are mostly off N % 16 / K % 512, so they take
the tile kernels. Here N is a multiple of 16 and K a multiple of 512, and M
runs from 1 to 520. That reaches every route of the staged last-rows kernel:
  * M <= 128: the one-row, LDS-streamed and staged kernels;
  * 129-512 rows: 128-row blocks of the staged kernel;
  * tiles plus the last rows above that.
Each SKU is routed separately: int8 / u8 RCR, s8 / u8 RRR and FP8 RCR / RRR.
The checks are those of test_gpu_sweep: bit-exact for integers, the FP8
tolerance of the other FP8 tests.
"""
import pytest

from oracle.inputs import rng
from tests import test_gpu_sweep as S
from baracuda_amd import plans as P

pytestmark = pytest.mark.gpu


def _row_grid_shapes(count, seed):
    g = rng(seed)
    out = []
    for i in range(count):
        m = int(g.integers(1, 129)) if i % 3 == 0 else int(g.integers(129, 521)) if i % 3 == 1 \
            else int(g.integers(1, 521))
        n = 16 * int(g.integers(1, 97))
        k = 512 * int(g.integers(1, 5))
        out.append((m, n, k))
    return out


ROWS = _row_grid_shapes(12, 4242)


@pytest.mark.parametrize("shape", ROWS)
def test_int8_rows_grid_sweep(gpu, shape):
    S.test_int8_sweep(gpu, shape, False)


@pytest.mark.parametrize("shape", ROWS)
def test_u8_rcr_rows_grid_sweep(gpu, shape):
    S.test_u8_rcr_sweep(gpu, shape)


@pytest.mark.parametrize("shape", ROWS)
def test_fp8_rows_grid_sweep(gpu, shape):
    S.test_fp8_sweep(gpu, shape)


@pytest.mark.parametrize("shape", ROWS)
def test_int8_rrr_rows_grid_sweep(gpu, shape):
    S.test_int8_rrr_bias_relu_sweep(gpu, shape)


@pytest.mark.parametrize("shape", ROWS)
def test_u8_rrr_rows_grid_sweep(gpu, shape):
    S.test_u8_rrr_sweep(gpu, shape, False)


@pytest.mark.parametrize("shape", ROWS[::2])
@pytest.mark.parametrize("fmt,layout", [("e4m3", P.LayoutSku.Rrr), ("e5m2", P.LayoutSku.Rcr)])
def test_fp8_out_rows_grid_sweep(gpu, shape, fmt, layout):
    S.test_fp8_out_with_c_sweep(gpu, shape, fmt, layout)
