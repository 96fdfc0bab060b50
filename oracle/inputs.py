"""Seeded synthetic inputs for the BASELINE.json configurations (test infrastructure).

One generator for every consumer (tests, smoke, bench's CPU leg):
numpy PCG64 seeded with the config index (1-5) unless a test passes its own.
"""
from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def int8_uniform(g, shape):
    """int8 uniform in [-127, 127]."""
    return g.integers(-127, 128, size=shape, dtype=np.int16).astype(np.int8)


def w8a8(m, n, k, seed=2):
    g = rng(seed)
    a = int8_uniform(g, (m, k))
    w = int8_uniform(g, (n, k))
    sa = g.uniform(0.005, 0.02, size=m).astype(np.float32)
    sw = g.uniform(0.001, 0.01, size=n).astype(np.float32)
    return a, w, sa, sw


def moe_routing(tokens, experts, topk, seed=5, s=1.1):
    """Top-k distinct experts per token; first pick Zipf(s) over ranks 1..E,
    later picks Zipf-weighted without replacement.  Returns
    (sorted_token_ids, expert_ids) with pair id = token*topk + slot."""
    g = rng(seed)
    p = 1.0 / np.arange(1, experts + 1) ** s
    p /= p.sum()
    choice = np.empty((tokens, topk), dtype=np.int32)
    for t in range(tokens):
        choice[t] = g.choice(experts, size=topk, replace=False, p=p)
    pair_expert = choice.reshape(-1)
    order = np.argsort(pair_expert, kind="stable").astype(np.int32)
    return order, pair_expert[order].astype(np.int32)
