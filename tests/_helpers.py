"""Shared seeded input/parameter recipes (following the reference tests)."""

from __future__ import annotations

import math

import numpy as np
import torch


def redraw_zero_params(module: torch.nn.Module, std: float = 0.02) -> torch.nn.Module:
    """Zero-initialised parameters re-drawn N(0, std) (test_triangle_multiplication.py:135-138)."""
    with torch.no_grad():
        for p in module.parameters():
            if torch.count_nonzero(p) == 0:
                p.normal_(0, std)
    return module


def randomize_params(module: torch.nn.Module, seed: int = 42) -> torch.nn.Module:
    """Every parameter ~ N(0, 1/sqrt(fan_in)) for matrices, N(1, 0.1)/N(0, 0.1) for LN."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in module.named_parameters():
            if p.ndim == 2:
                p.copy_(torch.randn(p.shape, generator=g) / math.sqrt(p.shape[-1]))
            elif name.endswith("weight"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(0.1 * torch.randn(p.shape, generator=g))
    return module


def state(module: torch.nn.Module) -> dict:
    return {k: v.detach().clone() for k, v in module.state_dict().items()}


# ----------------------------------------------------------------------------
# numpy brute force (small sizes only)
# ----------------------------------------------------------------------------
def np_ln(v: np.ndarray, w: np.ndarray, b: np.ndarray | None, eps: float = 1e-5) -> np.ndarray:
    mu = v.mean()
    var = ((v - mu) ** 2).mean()
    y = (v - mu) / np.sqrt(var + eps) * w
    return y + b if b is not None else y


def np_sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


def np_params(params: dict) -> dict:
    return {k: v.detach().double().numpy() for k, v in params.items()}


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double()
    b = b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.double() - b.double()).abs().max())
