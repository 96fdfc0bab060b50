"""Writes the committed golden fixtures of this path (run from the repo root).

The reference ships no golden files for this path, so these vectors are
computed here with independent library arithmetic (numpy int64 matmul), not
with the oracle they check:
  config1_s8_rcr_256.npz  A,B int8 U[-127,127] (PCG64 seed 1), C = A.B^T int32
  wte_gather.npz          the capture_replay_gather_gemv.rs:40-48 table (V=3,H=4)
                          with the :54-112 expectation row 0 = [1,2,3,4]
"""
from pathlib import Path
import sys

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle.inputs import int8_uniform, rng  # noqa: E402

OUT = Path(__file__).resolve().parent


def main():
    g = rng(1)
    a = int8_uniform(g, (256, 256))
    b = int8_uniform(g, (256, 256))
    c = (a.astype(np.int64) @ b.astype(np.int64).T).astype(np.int32)
    np.savez_compressed(OUT / "config1_s8_rcr_256.npz", a=a, b=b, c=c)
    v, h = 3, 4
    e = np.arange(v * h)
    table = (1 + 10 * (e // h) + (e % h)).astype(np.float32).reshape(v, h)
    np.savez_compressed(OUT / "wte_gather.npz", table=table, idx=np.array([0], np.uint32),
                        expected=np.array([[1, 2, 3, 4]], np.float32))


if __name__ == "__main__":
    main()
