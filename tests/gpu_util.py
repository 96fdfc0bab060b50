"""Helpers for the GPU parity tests: host<->device moves and tolerances."""
import numpy as np
import torch


def dev(a: np.ndarray, device="cuda:0") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host_bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 at |x| (8 significant bits)."""
    ax = np.abs(x).astype(np.float64)
    e = np.floor(np.log2(np.where(ax > 0, ax, 2.0 ** -126)))
    return np.exp2(np.maximum(e, -126) - 7)


def sync():
    torch.cuda.synchronize()
