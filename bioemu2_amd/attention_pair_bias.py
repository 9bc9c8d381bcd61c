"""Attention with pair bias on MI355X — drop-ins for ``AttentionPairBias`` and
``AttentionPairBiasSlidingWindow``.

Mirrors ``src/bioemu2/biomoa/ops/attention_pair_bias.py:42-225``: the same
constructor arguments, parameters and ``state_dict`` keys (``norm_s.*`` when
``initial_norm``, ``proj_qkv.weight``, ``proj_q_bias``, ``proj_g.weight``,
``norm_z.weight`` [+ ``norm_z.bias``], ``proj_z.weight``, ``proj_o.weight``),
the same ``forward(s, z, mask, multiplicity=1)`` signature and shape
assertions (:146-149), and the same masking (masked keys replaced by
``-inf = -1e6``, :184-190).  ``tile_size`` only bounded the reference's
materialised logits (:193-222); the flash kernel never materialises them, so
it is accepted and does not change the result.  ``use_efficient_fusion``
folds the LayerNorm gain into the projection in the reference (:118-126);
mathematically the same bias, so both settings run the same kernel.

``AttentionPairBiasSlidingWindow`` mirrors :228-340 (the denoiser's atom
transformer): constructor ``(c_s, c_z, num_heads, window_queries=32,
window_keys=128, inf, initial_norm, tile_size, zero_init_output,
use_bias_in_layer_norm)``, the same parameters, and
``forward(s [B*M*NW, W, c_s], z [B, NW, W, H, c_z], mask [B*NW, W], multiplicity)``.

Arithmetic follows the caller's precision: fp32 inputs with autocast off (the
reference's denoiser, score_model.py:355, model.py:387) run the fp32 path
(fp32 operands and accumulation, ``bioemu_apb_fwd_f32`` / ``bioemu_swa_fwd_f32``);
anything else runs bf16 MFMA operands with fp32 accumulation, as the
reference's bf16-autocast trunk.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from torch import Tensor

from . import _ops
from ._params import PreparedParams


class AttentionPairBias(nn.Module):
    def __init__(
        self,
        c_s: int,
        c_z: int,
        num_heads: int,
        inf: float = 1e6,
        initial_norm: bool = True,
        tile_size: int | None = 512,
        zero_init_output: bool = False,
        use_bias_in_layer_norm: bool = False,
        use_efficient_fusion: bool = False,
    ) -> None:
        super().__init__()
        assert c_s % num_heads == 0
        if use_efficient_fusion and use_bias_in_layer_norm:
            raise ValueError(
                "use_efficient_fusion=True is incompatible with use_bias_in_layer_norm=True: "
                "the LayerNorm+Linear fold cannot absorb a LayerNorm bias."
            )
        self.c_s = c_s
        self.c_z = c_z
        self.num_heads = num_heads
        self.head_dim = c_s // num_heads
        self.inf = inf
        self.tile_size = tile_size
        self.use_bias_in_layer_norm = use_bias_in_layer_norm
        self.use_efficient_fusion = use_efficient_fusion
        self.initial_norm = initial_norm
        if initial_norm:
            self.norm_s = nn.LayerNorm(c_s)
        self.proj_qkv = nn.Linear(c_s, 3 * c_s, bias=False)
        self.proj_q_bias = nn.Parameter(torch.zeros(c_s))
        self.proj_g = nn.Linear(c_s, c_s, bias=False)
        self.norm_z = nn.LayerNorm(c_z, bias=use_bias_in_layer_norm)
        self.proj_z = nn.Linear(c_z, num_heads, bias=False)
        self.proj_o = nn.Linear(c_s, c_s, bias=False)
        if zero_init_output:
            nn.init.zeros_(self.proj_o.weight)
        f32, bf = torch.float32, torch.bfloat16
        spec = []
        if initial_norm:
            spec += [("norm_s.weight", f32), ("norm_s.bias", f32)]
        spec += [("proj_qkv.weight", bf), ("proj_q_bias", f32), ("proj_g.weight", bf), ("norm_z.weight", f32)]
        if use_bias_in_layer_norm:
            spec += [("norm_z.bias", f32)]
        spec += [("proj_z.weight", bf), ("proj_o.weight", bf)]
        self._prepared = PreparedParams(spec)
        self._prepared32 = PreparedParams([(name, f32) for name, _ in spec])

    def _arrange(self, p: tuple[Tensor, ...]) -> tuple[Tensor | None, ...]:
        p = list(p)
        if not self.initial_norm:
            p = [None, None] + p
        if not self.use_bias_in_layer_norm:
            p.insert(6, None)
        return tuple(p)

    def prepared_params(self) -> tuple[Tensor | None, ...]:
        """(norm_s_w, norm_s_b, w_qkv, q_bias, w_g, norm_z_w, norm_z_b, w_z, w_o) in kernel dtypes."""
        return self._arrange(self._prepared.get(self))

    def prepared_params_f32(self) -> tuple[Tensor | None, ...]:
        """The same parameters, all fp32, for the fp32 arithmetic path."""
        return self._arrange(self._prepared32.get(self))

    def forward(self, s: Tensor, z: Tensor, mask: Tensor, multiplicity: int = 1) -> Tensor:
        assert s.ndim == 3 and z.ndim == 4 and mask.ndim == 2, f"{s.shape}, {z.shape}, {mask.shape}"
        assert s.shape[0] == z.shape[0] * multiplicity, f"{s.shape}, {z.shape}, multiplicity={multiplicity}"
        _ops.require_gpu(s, type(self).__name__)
        if self.inf != 1e6:
            raise ValueError("AttentionPairBias (HIP): only inf=1e6, the reference default, is supported")
        if _ops.fp32_mode(s):
            return torch.ops.bioemu_mi355x.attention_pair_bias_f32(
                s, z, _ops.mask_u8(mask), *self.prepared_params_f32(), self.num_heads, multiplicity
            )
        return torch.ops.bioemu_mi355x.attention_pair_bias(
            s, z, _ops.mask_u8(mask), *self.prepared_params(), self.num_heads, multiplicity
        )


class AttentionPairBiasSlidingWindow(AttentionPairBias):
    def __init__(
        self,
        c_s: int,
        c_z: int,
        num_heads: int,
        window_queries: int = 32,
        window_keys: int = 128,
        inf: float = 1e6,
        initial_norm: bool = True,
        tile_size: int | None = 512,
        zero_init_output: bool = False,
        use_bias_in_layer_norm: bool = False,
    ) -> None:
        super().__init__(
            c_s, c_z, num_heads, inf=inf, initial_norm=initial_norm, tile_size=tile_size,
            zero_init_output=zero_init_output, use_bias_in_layer_norm=use_bias_in_layer_norm,
        )
        self.window_queries = window_queries
        self.window_keys = window_keys

    def forward(self, s: Tensor, z: Tensor, mask: Tensor, multiplicity: int = 1) -> Tensor:
        assert s.ndim == 3 and z.ndim == 5 and mask.ndim == 2, f"{s.shape}, {z.shape}, {mask.shape}"
        _ops.require_gpu(s, type(self).__name__)
        if self.inf != 1e6:
            raise ValueError("AttentionPairBiasSlidingWindow (HIP): only inf=1e6, the reference default, is supported")
        if _ops.fp32_mode(s):
            return torch.ops.bioemu_mi355x.attention_pair_bias_sliding_window_f32(
                s, z, _ops.mask_u8(mask), *self.prepared_params_f32(), self.num_heads, multiplicity
            )
        return torch.ops.bioemu_mi355x.attention_pair_bias_sliding_window(
            s, z, _ops.mask_u8(mask), *self.prepared_params(), self.num_heads, multiplicity
        )
