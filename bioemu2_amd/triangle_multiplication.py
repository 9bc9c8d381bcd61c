"""Triangle multiplicative update on MI355X — drop-in for the reference TriMul variants.

Mirrors ``src/bioemu2/biomoa/ops/triangle_multiplication.py``:

* ``_TriMulBase`` has the same parameters and ``state_dict`` keys
  (:62-76): ``norm_in.{weight,bias}``, ``p_in.weight``, ``g_in.weight``,
  ``norm_out.{weight,bias}``, ``p_out.weight``, ``g_out.weight``.
* ``TriangleMultiplicationHip.forward(x, mask)`` computes what
  ``TriangleMultiplicationFull.forward`` (:89-99) does, with bf16 MFMA
  operands and fp32 accumulation, through one HIP kernel pipeline.
* ``REGISTRY`` maps every reference variant name (``full``, ``cueq``,
  ``cueq_tiled``) plus ``hip`` to the HIP class, so a checkpoint config
  selecting the CUDA-only ``cueq`` default runs unchanged on ROCm.
"""

from __future__ import annotations

import logging
from enum import Enum

import torch
import torch.nn as nn
from torch import Tensor

from . import _ops
from ._params import PreparedParams

logger = logging.getLogger(__name__)

_ACCEPTED_PRECISIONS = (None, "ieee", "tf32", "tf32x3", "highest", "high", "medium", "bf16")


class TriMulVariant(str, Enum):
    FULL = "full"
    CUEQ = "cueq"
    CUEQ_TILED = "cueq_tiled"
    HIP = "hip"


class _TriMulBase(nn.Module):
    """Shared weights (triangle_multiplication.py:62-76)."""

    def __init__(self, dim: int = 128, mode: str = "outgoing", **kwargs) -> None:
        super().__init__()
        assert mode in ("outgoing", "incoming")
        self.mode = mode
        self.dim = dim
        self.norm_in = nn.LayerNorm(dim, eps=1e-5)
        self.p_in = nn.Linear(dim, 2 * dim, bias=False)
        self.g_in = nn.Linear(dim, 2 * dim, bias=False)
        self.norm_out = nn.LayerNorm(dim)
        self.p_out = nn.Linear(dim, dim, bias=False)
        self.g_out = nn.Linear(dim, dim, bias=False)


_F32 = torch.float32
_BF16 = torch.bfloat16
TRIMUL_PARAM_SPEC = [
    ("norm_in.weight", _F32),
    ("norm_in.bias", _F32),
    ("p_in.weight", _BF16),
    ("g_in.weight", _BF16),
    ("norm_out.weight", _F32),
    ("norm_out.bias", _F32),
    ("p_out.weight", _BF16),
    ("g_out.weight", _BF16),
]


class TriangleMultiplicationHip(_TriMulBase):
    """HIP/gfx950 triangle multiplication (outgoing or incoming).

    Accepts the constructor kwargs of every reference variant
    (``dim, mode, tile_size, matmul_precision``).  ``tile_size`` is accepted
    for registry compatibility and unused (the kernels tile internally and
    keep N^2 scratch in HBM).  ``matmul_precision`` is validated and
    recorded.  bf16 inputs, or fp32 inputs under bf16 autocast (the
    reference trunk's policy), run the bf16 path: bf16 MFMA operands, fp32
    accumulation, output in x's dtype.  fp32 inputs with autocast off run
    IEEE fp32 arithmetic throughout (``bioemu_trimul_fwd_f32``), as the
    reference's ``"ieee"`` default and TriangleMultiplicationFull's fp32
    einsum do (triangle_multiplication.py:94, :117).  Inference only: there is
    no backward.
    """

    def __init__(
        self,
        dim: int = 128,
        mode: str = "outgoing",
        tile_size: int | None = None,
        matmul_precision: str | None = None,
    ) -> None:
        super().__init__(dim, mode)
        if matmul_precision not in _ACCEPTED_PRECISIONS:
            raise ValueError(
                f"TriangleMultiplicationHip matmul_precision must be one of "
                f"{_ACCEPTED_PRECISIONS}; got {matmul_precision!r}."
            )
        self.tile_size = tile_size
        self._matmul_precision = matmul_precision
        self._prepared = PreparedParams(TRIMUL_PARAM_SPEC)
        self._prepared32 = PreparedParams([(name, _F32) for name, _ in TRIMUL_PARAM_SPEC])

    def prepared_params(self) -> tuple[Tensor, ...]:
        return self._prepared.get(self)

    def prepared_params_f32(self) -> tuple[Tensor, ...]:
        return self._prepared32.get(self)

    def forward(self, x: Tensor, mask: Tensor) -> Tensor:
        _ops.require_gpu(x, type(self).__name__)
        if _ops.fp32_mode(x):
            return torch.ops.bioemu_mi355x.trimul_f32(
                x, _ops.mask_u8(mask), *self.prepared_params_f32(), self.mode == "outgoing"
            )
        return torch.ops.bioemu_mi355x.trimul(
            x, _ops.mask_u8(mask), *self.prepared_params(), self.mode == "outgoing"
        )


class TriangleMultiplicationOutgoing(TriangleMultiplicationHip):
    """``TriangleMultiplicationOutgoing(dim)`` (triangle_multiplication.py:370-381)."""

    def __init__(self, dim: int = 128) -> None:
        super().__init__(dim=dim, mode="outgoing")


class TriangleMultiplicationIncoming(TriangleMultiplicationHip):
    """``TriangleMultiplicationIncoming(dim)`` (triangle_multiplication.py:384-395)."""

    def __init__(self, dim: int = 128) -> None:
        super().__init__(dim=dim, mode="incoming")


# Registry mapping TriMulVariant -> (module_path, class_name); same shape as
# the reference REGISTRY (triangle_multiplication.py:348-352).
REGISTRY: dict[TriMulVariant, tuple[str, str]] = {
    TriMulVariant.FULL: (__name__, "TriangleMultiplicationHip"),
    TriMulVariant.CUEQ: (__name__, "TriangleMultiplicationHip"),
    TriMulVariant.CUEQ_TILED: (__name__, "TriangleMultiplicationHip"),
    TriMulVariant.HIP: (__name__, "TriangleMultiplicationHip"),
}
