"""Triangle attention (starting / ending node) on MI355X.

The reference has no triangle attention: its trunk is a PairMixer stack that
removes it (``src/bioemu2/biomoa/modules/pairmixer.py:459-462``).  These
modules restate AlphaFold3 supplement Alg. 14/15 with LinearNoBias
projections and the reference's attention masking convention (masked keys
are replaced by ``-inf = -1e6`` before the softmax,
``src/bioemu2/biomoa/ops/attention_pair_bias.py:184-190``).

They plug into the reference's variant factory through its 3-tuple registry
form ``(module, starting_class, ending_class)`` selected by ``starting=``
(``src/bioemu2/biomoa/utils/strategy.py:33-36``): see ``REGISTRY``.

Parameters (``state_dict`` keys): ``norm.{weight,bias}``,
``proj_q/proj_k/proj_v/proj_g.weight [H*d, c]``, ``proj_b.weight [H, c]``,
``proj_o.weight [c, H*d]``.
"""

from __future__ import annotations

from enum import Enum

import torch
import torch.nn as nn
from torch import Tensor

from . import _ops
from ._params import PreparedParams


class TriAttVariant(str, Enum):
    HIP = "hip"


class _PackedTriAttParams(PreparedParams):
    """norm fp32; [Wq; Wk; Wv; Wg; Wb] packed and Wo in ``dtype`` (bf16, or fp32 for the fp32 path)."""

    def __init__(self, dtype: torch.dtype = torch.bfloat16):
        super().__init__(
            [("norm.weight", torch.float32), ("norm.bias", torch.float32)]
            + [(f"proj_{n}.weight", dtype) for n in ("q", "k", "v", "g", "b", "o")]
        )

    def get(self, module: nn.Module) -> tuple[Tensor, ...]:
        key_before = self._key
        val = super().get(module)
        if self._key != key_before or not hasattr(self, "_packed"):
            nw, nb, wq, wk, wv, wg, wb, wo = val
            self._packed = (nw, nb, torch.cat([wq, wk, wv, wg, wb], dim=0).contiguous(), wo)
        return self._packed


class TriangleAttentionHip(nn.Module):
    """Triangle attention around the starting (``starting=True``) or ending node.

    ``forward(z [B,N,N,c], mask [B,N,N]) -> [B,N,N,c]`` returns the update
    (callers add the residual, as ``PairMixerLayer.forward`` does for its ops,
    pairmixer.py:446-456).  bf16 operands, fp32 accumulation and softmax; fp32
    inputs with autocast off (the reference's fp32 mode) compute in fp32
    throughout.  Supported: c = 128 with 4 heads of 32 (fp32: also c = 32, one
    head).  Inference only.
    """

    def __init__(
        self,
        c_z: int = 128,
        num_heads: int = 4,
        starting: bool = True,
        inf: float = 1e6,
        matmul_precision: str | None = None,
        **kwargs,
    ) -> None:
        super().__init__()
        if c_z % num_heads:
            raise ValueError(f"c_z={c_z} not divisible by num_heads={num_heads}")
        self.c_z = c_z
        self.num_heads = num_heads
        self.head_dim = c_z // num_heads
        self.starting = starting
        self.inf = inf
        self.norm = nn.LayerNorm(c_z)
        hd = num_heads * self.head_dim
        self.proj_q = nn.Linear(c_z, hd, bias=False)
        self.proj_k = nn.Linear(c_z, hd, bias=False)
        self.proj_v = nn.Linear(c_z, hd, bias=False)
        self.proj_g = nn.Linear(c_z, hd, bias=False)
        self.proj_b = nn.Linear(c_z, num_heads, bias=False)
        self.proj_o = nn.Linear(hd, c_z, bias=False)
        self._prepared = _PackedTriAttParams()
        self._prepared32 = _PackedTriAttParams(torch.float32)

    def prepared_params(self) -> tuple[Tensor, ...]:
        return self._prepared.get(self)

    def prepared_params_f32(self) -> tuple[Tensor, ...]:
        """The same packed parameters, all fp32, for the fp32 arithmetic path."""
        return self._prepared32.get(self)

    def forward(self, z: Tensor, mask: Tensor) -> Tensor:
        _ops.require_gpu(z, type(self).__name__)
        if self.inf != 1e6:
            raise ValueError("TriangleAttentionHip: only inf=1e6 (the reference masking value) is supported")
        if _ops.fp32_mode(z):
            return torch.ops.bioemu_mi355x.triangle_attention_f32(
                z, _ops.mask_u8(mask), *self.prepared_params_f32(), self.starting, self.num_heads
            )
        return torch.ops.bioemu_mi355x.triangle_attention(
            z, _ops.mask_u8(mask), *self.prepared_params(), self.starting, self.num_heads
        )


class TriangleAttentionStartingNodeHip(TriangleAttentionHip):
    def __init__(self, c_z: int = 128, num_heads: int = 4, **kwargs) -> None:
        kwargs.pop("starting", None)
        super().__init__(c_z, num_heads, starting=True, **kwargs)


class TriangleAttentionEndingNodeHip(TriangleAttentionHip):
    def __init__(self, c_z: int = 128, num_heads: int = 4, **kwargs) -> None:
        kwargs.pop("starting", None)
        super().__init__(c_z, num_heads, starting=False, **kwargs)


# 3-tuple registry entries: make(REGISTRY, "hip", starting=True|False, ...)
REGISTRY: dict[TriAttVariant, tuple[str, str, str]] = {
    TriAttVariant.HIP: (__name__, "TriangleAttentionStartingNodeHip", "TriangleAttentionEndingNodeHip"),
}
