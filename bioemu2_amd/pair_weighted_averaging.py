"""Pair-weighted averaging on MI355X — drop-in for the reference MSA-module op.

Mirrors ``src/bioemu2/biomoa/ops/pair_weighted_averaging.py``: the
``PairWeightedAveraging(c_m, c_z, c_h, num_heads, inf=1e6,
use_bias_in_layer_norm=True)`` constructor (:9-57), its parameters and
``state_dict`` keys (``norm_m.{weight,bias}``, ``norm_z.weight[, norm_z.bias]``,
``proj_m.weight``, ``proj_g.weight``, ``proj_z.weight``, ``proj_o.weight``) and
``forward(m [B,S,N,c_m], z [B,N,N,c_z], mask [B,N,N], chunk_heads=False) ->
[B,S,N,c_m]`` (:59-154).  ``chunk_heads`` only bounded the reference's peak
memory (both of its paths compute the same values); the HIP path never
materialises the per-head [B,H,S,N,c_h] tensors, so it is accepted and unused.

The bf16 kernels support the reference trunk's widths (PairMixerMSALayer,
biomoa/modules/pairmixer.py:673-678): c_m = 64, c_z = 128, c_h = 32, 8 heads.
fp32 inputs with autocast off (a ``--precision 32-true`` run) take the IEEE
fp32 entry point ``bioemu_pwa_fwd_f32`` (c_h = 32; c_m a multiple of 32; any
head count and ``inf``); fp32 inputs under bf16 autocast take the bf16 path.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from torch import Tensor

from . import _ops
from ._params import PreparedParams


class PairWeightedAveraging(nn.Module):
    def __init__(
        self,
        c_m: int,
        c_z: int,
        c_h: int,
        num_heads: int,
        inf: float = 1e6,
        use_bias_in_layer_norm: bool = True,
    ) -> None:
        super().__init__()
        self.c_m = c_m
        self.c_z = c_z
        self.c_h = c_h
        self.num_heads = num_heads
        self.inf = inf
        self.use_bias_in_layer_norm = use_bias_in_layer_norm
        self.norm_m = nn.LayerNorm(c_m)
        self.norm_z = nn.LayerNorm(c_z, bias=use_bias_in_layer_norm)
        self.proj_m = nn.Linear(c_m, c_h * num_heads, bias=False)
        self.proj_g = nn.Linear(c_m, c_h * num_heads, bias=False)
        self.proj_z = nn.Linear(c_z, num_heads, bias=False)
        self.proj_o = nn.Linear(c_h * num_heads, c_m, bias=False)
        f32, bf = torch.float32, torch.bfloat16
        spec = [("norm_m.weight", f32), ("norm_m.bias", f32), ("proj_m.weight", bf), ("proj_g.weight", bf),
                ("norm_z.weight", f32)]
        if use_bias_in_layer_norm:
            spec.append(("norm_z.bias", f32))
        spec += [("proj_z.weight", bf), ("proj_o.weight", bf)]
        self._prepared = PreparedParams(spec)
        self._prepared32 = PreparedParams([(name, f32) for name, _ in spec])

    def _arrange(self, p: tuple[Tensor, ...]) -> tuple[Tensor | None, ...]:
        return p if self.use_bias_in_layer_norm else p[:5] + (None,) + p[5:]

    def prepared_params(self) -> tuple[Tensor | None, ...]:
        """(norm_m.w, norm_m.b, w_m, w_g, norm_z.w, norm_z.b or None, w_z, w_o) on the device."""
        return self._arrange(self._prepared.get(self))

    def prepared_params_f32(self) -> tuple[Tensor | None, ...]:
        """The same parameters, all fp32, for the fp32 arithmetic path."""
        return self._arrange(self._prepared32.get(self))

    def forward(self, m: Tensor, z: Tensor, mask: Tensor, chunk_heads: bool = False) -> Tensor:
        _ops.require_gpu(m, type(self).__name__)
        if _ops.fp32_mode(m):
            return torch.ops.bioemu_mi355x.pair_weighted_averaging_f32(
                m, z, mask, *self.prepared_params_f32(), self.num_heads, float(self.inf))
        if self.inf != 1e6:
            raise ValueError(f"PairWeightedAveraging: only inf=1e6 is supported (got {self.inf})")
        return torch.ops.bioemu_mi355x.pair_weighted_averaging(m, z, mask, *self.prepared_params(), self.num_heads)
