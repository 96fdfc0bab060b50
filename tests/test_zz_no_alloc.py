"""The allocation-free u8 RRR entry point (baracuda_kernels_gemm_u8_rrr_gfx950_noalloc_run)
against the workspace entry point it is a variant of, through the C ABI.

Two calls in a row on one device (the second smaller, so it runs on what the
first left in the shared scratch), each compared byte for byte with
baracuda_kernels_gemm_u8_rrr_gfx950_run given a caller workspace filled with
garbage; the oversize rejection; and a ragged shape that never touches the
scratch.  The u8 result itself is pinned against an int64 matmul.
"""
import ctypes

import numpy as np
import pytest
import torch

from baracuda_amd import ffi
from oracle.inputs import rng
from tests.gpu_util import dev, sync

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20   # BARACUDA_U8_RRR_NOALLOC_SCRATCH_BYTES


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _inputs(m, n, k, seed):
    g = rng(seed)
    a = dev(g.integers(0, 256, (m, k), dtype=np.uint8))
    b = dev(g.integers(0, 256, (k, n), dtype=np.uint8))
    c = dev(g.integers(0, 256, (m, n), dtype=np.uint8))
    return a, b, c


def _noalloc(L, a, b, c, alpha, beta):
    m, k = a.shape
    n = b.shape[1]
    d = torch.full((m, n), 7, dtype=torch.uint8, device=a.device)
    st = L.gemm_u8_rrr_gfx950_noalloc_run(m, n, k, _p(a), k, _p(b), n, _p(c), n, _p(d), n, alpha, beta, None)
    return st, d


def _with_workspace(L, a, b, c, alpha, beta):
    m, k = a.shape
    n = b.shape[1]
    wsb = L.gemm_u8_rrr_gfx950_workspace_size(m, n, k)
    ws = torch.full((max(wsb, 1),), 0xAB, dtype=torch.uint8, device=a.device)
    d = torch.full((m, n), 9, dtype=torch.uint8, device=a.device)
    st = L.gemm_u8_rrr_gfx950_run(m, n, k, _p(a), k, _p(b), n, _p(c), n, _p(d), n, alpha, beta,
                                  _p(ws), wsb, None)
    return st, d, wsb


def test_noalloc_matches_workspace_entry_two_calls(gpu):
    L = ffi.lib()
    alpha, beta = 1.0 / (1 << 17), 0.5
    # first call larger than the second: the second runs over the first's scratch contents
    for (m, n, k), seed in (((1024, 768, 1024), 71), ((512, 256, 384), 72)):
        print(f"noalloc u8 rrr m={m} n={n} k={k} seed={seed}", flush=True)
        a, b, c = _inputs(m, n, k, seed)
        st_ref, want, wsb = _with_workspace(L, a, b, c, alpha, beta)
        assert st_ref == 0 and wsb > 0
        st, got = _noalloc(L, a, b, c, alpha, beta)
        assert st == 0
        sync()
        assert torch.equal(got, want)
        # ... and both equal sat_u8(rne(alpha*acc + beta*c)) from an exact int64 product
        acc = (a.cpu().to(torch.int64) @ b.cpu().to(torch.int64)).numpy()
        y = np.float32(alpha) * acc.astype(np.float32) + np.float32(beta) * c.cpu().numpy().astype(np.float32)
        assert np.array_equal(got.cpu().numpy(), np.clip(np.rint(y), 0, 255).astype(np.uint8))


def test_noalloc_rejects_oversize_and_runs_ragged(gpu):
    L = ffi.lib()
    # 4096 x 4096 x 8192: 64 MiB of flipped operands + the sums > the scratch
    m, n, k = 4096, 4096, 8192
    assert L.gemm_u8_rrr_gfx950_workspace_size(m, n, k) > SCRATCH_BYTES
    a = torch.zeros((m, k), dtype=torch.uint8, device=gpu)
    b = torch.zeros((k, n), dtype=torch.uint8, device=gpu)
    d = torch.zeros((m, n), dtype=torch.uint8, device=gpu)
    st = L.gemm_u8_rrr_gfx950_noalloc_run(m, n, k, _p(a), k, _p(b), n, None, n, _p(d), n, 1.0, 0.0, None)
    assert st == 4
    del a, b, d
    # a ragged shape takes the in-loop path (no scratch), same bytes as the workspace entry
    a, b, c = _inputs(300, 520, 200, 73)
    st_ref, want, _ = _with_workspace(L, a, b, c, 0.01, 0.25)
    st, got = _noalloc(L, a, b, c, 0.01, 0.25)
    sync()
    assert st_ref == 0 and st == 0 and torch.equal(got, want)
