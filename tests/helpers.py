"""Shared test helpers: tolerances, comparisons, seeded inputs."""
from __future__ import annotations

import numpy as np
import torch

# bf16 outputs vs an fp32 reference (stated tolerance of the path)
BF16_MAX_ABS = 2e-2
BF16_MEAN_ABS = 2e-3
FP8_COSINE = 0.999


def diff_stats(a: torch.Tensor, b: torch.Tensor):
    d = (a.detach().float().cpu() - b.detach().float().cpu()).abs()
    return d.max().item(), d.mean().item()


def cosine(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu().flatten()
    b = b.detach().double().cpu().flatten()
    return float((a @ b) / (a.norm() * b.norm()))


def assert_bf16_close(out: torch.Tensor, ref: torch.Tensor, what: str = "",
                      max_abs: float = BF16_MAX_ABS, mean_abs: float = BF16_MEAN_ABS):
    mx, mn = diff_stats(out, ref)
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max-abs {mx:.3e} (<= {max_abs}), mean-abs {mn:.3e} (<= {mean_abs})"


def gen(seed: int):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def randn(shape, g, dtype=torch.float32, scale=1.0):
    return (torch.randn(shape, generator=g, dtype=torch.float32) * scale).to(dtype)


def bf16_ulp_diff(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    """Distance in bf16 units-in-the-last-place between two bf16 tensors."""
    ai = a.detach().cpu().contiguous().view(torch.int16).numpy().astype(np.int32)
    bi = b.detach().cpu().contiguous().view(torch.int16).numpy().astype(np.int32)
    # map sign-magnitude to a monotone integer line
    ai = np.where(ai < 0, -(ai & 0x7FFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFF), bi)
    return np.abs(ai - bi)
