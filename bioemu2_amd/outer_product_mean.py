"""Fused OuterProductMean on MI355X — drop-in for the reference OPM variants.

Mirrors ``src/bioemu2/biomoa/ops/outer_product_mean.py``: ``_OPMBase``
parameters and ``state_dict`` keys (:32-39: ``norm.{weight,bias}``,
``proj_ab.weight``, ``proj_o.{weight,bias}``), the
``forward(m [B,S,N,C_in], mask [B,S,N] | [B,N]) -> [B,N,N,C_out]`` contract
of ``OuterProductMeanVanilla`` (:45-75) with its divisor (valid-row count per
batch for a 3-D mask, 1 for a 2-D mask), and a ``REGISTRY`` keyed by the
reference's ``OPMVariant`` values so ``make(REGISTRY, "vanilla" |
"triton_memory_saving", ...)`` resolves to the HIP class.  ``tile_size``
bounded the reference's memory (:23, :107-127); the fused kernel never
materialises the [N,N,C_H^2] intermediate, so it is accepted and unused.
fp32 inputs with autocast off (a ``--precision 32-true`` run) take the IEEE
fp32 entry point ``bioemu_opm_fwd_f32`` (LayerNorm, projections, contraction,
mean and proj_o all fp32; c_hidden = 32); fp32 inputs under bf16 autocast take
the bf16 path, whose contraction accumulates in fp32 as the reference's
forced-fp32 einsum does (:64-74).
"""

from __future__ import annotations

from enum import Enum

import torch
import torch.nn as nn
from torch import Tensor

from . import _ops
from ._params import PreparedParams

_DEFAULT_TILE_SIZE = 256


class OPMVariant(str, Enum):
    VANILLA = "vanilla"
    TRITON_MEMORY_SAVING = "triton_memory_saving"
    HIP = "hip"


class OuterProductMeanHip(nn.Module):
    def __init__(
        self,
        c_in: int,
        c_hidden: int,
        c_out: int,
        tile_size: int | None = None,
        matmul_precision: str | None = None,
    ) -> None:
        super().__init__()
        self.c_hidden = c_hidden
        self.tile_size = _DEFAULT_TILE_SIZE if tile_size is None else tile_size
        self.norm = nn.LayerNorm(c_in)
        self.proj_ab = nn.Linear(c_in, 2 * c_hidden, bias=False)
        self.proj_o = nn.Linear(c_hidden * c_hidden, c_out)
        f32, bf = torch.float32, torch.bfloat16
        self._prepared = PreparedParams(
            [("norm.weight", f32), ("norm.bias", f32), ("proj_ab.weight", bf), ("proj_o.weight", bf),
             ("proj_o.bias", f32)]
        )
        self._prepared32 = PreparedParams(
            [(name, f32) for name in ("norm.weight", "norm.bias", "proj_ab.weight", "proj_o.weight", "proj_o.bias")]
        )

    def prepared_params(self) -> tuple[Tensor, ...]:
        return self._prepared.get(self)

    def prepared_params_f32(self) -> tuple[Tensor, ...]:
        """The same parameters, all fp32, for the fp32 arithmetic path."""
        return self._prepared32.get(self)

    def forward(self, m: Tensor, mask: Tensor) -> Tensor:
        _ops.require_gpu(m, type(self).__name__)
        if _ops.fp32_mode(m):
            return torch.ops.bioemu_mi355x.outer_product_mean_f32(m, mask, *self.prepared_params_f32())
        return torch.ops.bioemu_mi355x.outer_product_mean(m, mask, *self.prepared_params())


REGISTRY: dict[OPMVariant, tuple[str, str]] = {
    OPMVariant.VANILLA: (__name__, "OuterProductMeanHip"),
    OPMVariant.TRITON_MEMORY_SAVING: (__name__, "OuterProductMeanHip"),
    OPMVariant.HIP: (__name__, "OuterProductMeanHip"),
}
