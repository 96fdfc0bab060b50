"""Seeded random-shape sweep over the int8 weight-only GEMV and the grouped
int8 MoE GEMM (GPU parity; the bars of test_gpu_decode / test_gpu_moe)."""
import numpy as np
import pytest

from oracle.inputs import rng
from tests.test_gpu_decode import _gemv_check, _gemv_inputs, _gemv_run
from tests.test_gpu_moe import _block_routing, _run as _moe_run

pytestmark = pytest.mark.gpu


def _gemv_shapes(count, seed):
    g = rng(seed)
    out = []
    for i in range(count):
        n = int(g.integers(1, 5000))
        k = int(g.integers(1, 9)) * 1024 if i % 2 else int(g.integers(1, 6000))
        out.append((n, k))
    return out


@pytest.mark.parametrize("shape", _gemv_shapes(16, 77))
def test_gemv_s8w_sweep(gpu, shape):
    print(f"case: sweep gemv_s8w {shape}", flush=True)
    w, scale, xb = _gemv_inputs(*shape, seed=shape[0] + shape[1])
    _gemv_check(_gemv_run(w, scale, xb), w, scale, xb)


def _moe_cases(count, seed):
    g = rng(seed)
    out = []
    for i in range(count):
        e = int(g.integers(1, 20))
        counts = [int(c) for c in g.integers(0, 600, e)]
        if sum(counts) == 0:
            counts[0] = 1
        n = int(g.integers(1, 4)) * 256 if i % 3 else int(g.integers(16, 700))
        k = int(g.integers(1, 6)) * 128 if i % 2 else int(g.integers(8, 700))
        out.append((counts, n, k, seed + i))
    return out


@pytest.mark.parametrize("case", _moe_cases(12, 300))
def test_moe_sweep(gpu, case):
    # top-1 block routing with random per-expert row counts (empty experts,
    # partial last tiles), N / K on and off the LDS-DMA grid; every pair.
    counts, n, k, seed = case
    print(f"case: sweep moe E={len(counts)} rows={sum(counts)} n={n} k={k}", flush=True)
    tokens, routing = _block_routing(counts, seed=seed)
    _moe_run(tokens=tokens, E=len(counts), topk=1, n=n, k=k, seed=seed, routing=routing)


def _moe_decode_cases(count, seed):
    # at most 64 pairs: the decode kernels (staged, and the dot4 row kernel
    # for 3-6 pairs with K % 1024 == 0); K on the 512 / 1024 grids and off
    # them (the tile path)
    g = rng(seed)
    out = []
    for i in range(count):
        e = int(g.integers(1, 17))
        cap = 8 if i % 3 == 0 else 64
        counts = [0] * e
        for _ in range(int(g.integers(1, cap + 1))):
            counts[int(g.integers(0, e))] += 1
        n = int(g.integers(1, 5)) * 256
        k = (int(g.integers(1, 5)) * 1024 if i % 4 != 3 else int(g.integers(1, 9)) * 512) if i % 5 else \
            int(g.integers(1, 20)) * 128
        out.append((counts, n, k, seed + i))
    return out


@pytest.mark.parametrize("case", _moe_decode_cases(15, 401))
def test_moe_decode_sweep(gpu, case):
    # decode-sized routing (empty experts, one expert with many rows), every
    # pair bit-exact, the counts and offsets the decode kernels write
    counts, n, k, seed = case
    print(f"case: sweep moe decode E={len(counts)} rows={sum(counts)} n={n} k={k}", flush=True)
    tokens, routing = _block_routing(counts, seed=seed)
    _moe_run(tokens=tokens, E=len(counts), topk=1, n=n, k=k, seed=seed, routing=routing)
