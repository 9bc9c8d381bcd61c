"""SwiGLU Transition on MI355X — drop-in for ``src/bioemu2/biomoa/ops/transition.py``.

Same constructor (``dim, hidden, out_dim, use_norm, chunk_size``), parameters
and ``state_dict`` keys (``norm.{weight,bias}`` when ``use_norm``,
``fc1.weight``, ``fc2.weight``, ``fc3.weight``; transition.py:34-50) and the
same result ``fc3(silu(fc1(LN x)) * fc2(LN x))`` (:52-76).  Rows of width 128
(hidden 512: the pair representation) or 64 (hidden 256: the MSA
representation) run one fused HIP kernel; other widths (the single
representation, 384) and ``out_dim != dim`` (the denoiser's token/atom
mixers, diffusion.py:623-634: dim a multiple of 16, hidden and out_dim
multiples of 32) run the token LN + GEMM kernels.
``chunk_size`` only tiled the hidden dimension for memory in the reference
(:76-91): the fused kernel never materialises the hidden activations, so it
is accepted and has no effect on the result.  fp32 inputs with autocast off
(the reference's denoiser) run the fp32 path (``bioemu_transition_fwd_f32``:
fp32 operands and accumulation, any row count; dim a multiple of 8).
"""

from __future__ import annotations

import torch
import torch.nn as nn
from torch import Tensor

from . import _ops
from ._params import PreparedParams


class Transition(nn.Module):
    def __init__(
        self,
        dim: int,
        hidden: int,
        out_dim: int | None = None,
        use_norm: bool = True,
        chunk_size: int | None = None,
    ) -> None:
        super().__init__()
        out_dim = out_dim or dim
        self.out_dim = out_dim
        self.use_norm = use_norm
        self.chunk_size = chunk_size
        if use_norm:
            self.norm = nn.LayerNorm(dim, eps=1e-5)
        self.fc1 = nn.Linear(dim, hidden, bias=False)
        self.fc2 = nn.Linear(dim, hidden, bias=False)
        self.fc3 = nn.Linear(hidden, out_dim, bias=False)
        self.hidden = hidden
        spec = [("fc1.weight", torch.bfloat16), ("fc2.weight", torch.bfloat16), ("fc3.weight", torch.bfloat16)]
        if use_norm:
            spec = [("norm.weight", torch.float32), ("norm.bias", torch.float32)] + spec
        self._prepared = PreparedParams(spec)
        self._prepared32 = PreparedParams([(name, torch.float32) for name, _ in spec])

    def prepared_params(self) -> tuple[Tensor | None, ...]:
        p = self._prepared.get(self)
        return p if self.use_norm else (None, None) + p

    def prepared_params_f32(self) -> tuple[Tensor | None, ...]:
        p = self._prepared32.get(self)
        return p if self.use_norm else (None, None) + p

    def forward(self, x: Tensor) -> Tensor:
        _ops.require_gpu(x, type(self).__name__)
        if _ops.fp32_mode(x):
            return torch.ops.bioemu_mi355x.transition_f32(x, *self.prepared_params_f32())
        return torch.ops.bioemu_mi355x.transition(x, *self.prepared_params())
