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


# ----------------------------------------------------------------------------
# Residual-tail format, restated in numpy (the statement the HIP split/join and
# every residual epilogue are checked against): value = hi + t * 2^(E(hi) - 142)
# with hi = round-to-nearest-even bf16 of the value, E its biased exponent
# field, t = clamp(rint((value - hi) * 2^(142 - E)), -127, 127).
# ----------------------------------------------------------------------------
def np_bf16_rne(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even (finite inputs)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def np_bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def np_tail_encode(v: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    v = np.asarray(v, dtype=np.float32)
    hi = np_bf16_rne(v)
    e = ((hi >> 7) & 0xFF).astype(np.int32)
    r = (v - np_bf16_to_f32(hi)).astype(np.float32)
    t = np.clip(np.rint(np.ldexp(r.astype(np.float64), 142 - e)), -127, 127).astype(np.int8)
    return hi, t


def np_tail_decode(hi: np.ndarray, t: np.ndarray) -> np.ndarray:
    e = ((hi >> 7) & 0xFF).astype(np.int32)
    return (np_bf16_to_f32(hi).astype(np.float64) + np.ldexp(t.astype(np.float64), e - 142)).astype(np.float32)
