"""GPU parity of EmbeddingPlan (embedding forward) against the CPU oracle.

Bar: bit-exact (a pure copy) for f32 / f64 / f16 / bf16 weights with i32
and i64 indices, padding_idx, negative and out-of-range indices, ragged row
lengths (element path) and more rows than one grid dimension holds.
"""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from oracle import oracle as O
from oracle.inputs import rng
from tests.gpu_util import sync

pytestmark = pytest.mark.gpu

DT = {torch.float32: np.float32, torch.float64: np.float64, torch.float16: np.float16,
      torch.bfloat16: np.uint16}


def _run(w, idx, pad):
    V, D = w.shape
    n = idx.numel()
    plan = P.EmbeddingPlan.select(P.EmbeddingDescriptor(V, D, n, pad, P._EMBED_KIND[w.dtype]))
    out = torch.full((n, D), 7, dtype=w.dtype, device="cuda:0")
    plan.run(w, idx, out)
    sync()
    return out


def _host(t):
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


@pytest.mark.parametrize("dtype", list(DT))
@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("shape", [(5, 4, 3), (32000, 4096, 1), (1000, 333, 70), (128, 8, 70000)])
def test_embedding_matches_oracle(gpu, dtype, idx_dtype, shape):
    V, D, n = shape
    print(f"case: embedding {dtype} {idx_dtype} {shape}", flush=True)
    g = rng(V + D + n)
    w = torch.from_numpy(g.standard_normal((V, D)).astype(np.float32)).to(dtype).to("cuda:0")
    idx_np = g.integers(-3, V + 3, n).astype(np.int64)
    idx_np[: min(n, 4)] = [0, V - 1, -1, V][: min(n, 4)]
    pad = int(idx_np[n // 2]) if n > 2 else None
    idx = torch.from_numpy(idx_np).to(idx_dtype).to("cuda:0")
    got = _host(_run(w, idx, pad))
    want = O.embedding(_host(w), idx_np.astype(np.int32 if idx_dtype == torch.int32 else np.int64), pad)
    assert got.tobytes() == want.tobytes()


def test_embedding_misaligned_base_and_empty(gpu):
    # A weight view starting 2 bytes into its buffer takes the element path.
    base = torch.randn(65 * 64 + 1, device="cuda:0").to(torch.bfloat16)
    w = base[1:].view(65, 64)
    idx = torch.tensor([3, 64, 0, 65], dtype=torch.int32, device="cuda:0")
    got = _host(_run(w, idx, None))
    want = O.embedding(_host(w), idx.cpu().numpy(), None)
    assert got.tobytes() == want.tobytes()
    # N == 0 and D == 0 are no-ops
    _run(torch.zeros((4, 8), device="cuda:0"), torch.zeros(0, dtype=torch.int32, device="cuda:0"), None)
    _run(torch.zeros((4, 0), device="cuda:0"), torch.zeros(3, dtype=torch.int32, device="cuda:0"), None)
